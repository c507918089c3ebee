"""Checks that pin the C oracle (oracle/ccv1d_oracle.c) to what the mathematics and the reference's
definition fix. Each check returns (ok, detail) so that tests/test_oracle.py can assert on it and
tests/test_oracle_mutations.py can show that a planted mistake makes at least one of them fail.
"""

import json
import os

import numpy as np
import torch

import ccv1d_oracle as oracle
import closed_form as cf

_KAT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kat_exact.json")


def make_case(seed, B, T, D, W, bias=True, init=False, seq=None, dfinal=False, silu=True,
              w_scale=None):
    """Random float32 CPU tensors. seq: None | "segments" | "equal" | "distinct" | "padded"."""
    g = torch.Generator().manual_seed(seed)
    P = W - 1
    c = {"B": B, "T": T, "D": D, "W": W, "silu": silu}
    c["x"] = torch.randn(B, T, D, generator=g)
    c["w"] = torch.randn(D, W, generator=g) * (w_scale if w_scale else 1.0 / W ** 0.5)
    c["b"] = torch.randn(D, generator=g) if bias else None
    c["init"] = torch.randn(B, P, D, generator=g) if init else None
    c["dout"] = torch.randn(B, T, D, generator=g)
    c["dfinal"] = torch.randn(B, P, D, generator=g) if dfinal else None
    if seq is None:
        c["seq"] = None
    elif seq == "equal":
        c["seq"] = torch.full((B, T), 3, dtype=torch.int32)
    elif seq == "distinct":
        c["seq"] = torch.arange(B * T, dtype=torch.int32).reshape(B, T) + 1
    else:
        s = torch.zeros(B, T, dtype=torch.int32)
        for b in range(B):
            t, sid = 0, 0
            while t < T:
                n = int(torch.randint(1, max(2, T // 3) + 1, (1,), generator=g))
                s[b, t:t + n] = sid
                t += n
                sid += 1
            if seq == "padded":
                npad = max(1, T // 5)
                s[b, T - npad:] = -1
                if T > 4:
                    s[b, T // 2] = -2
        c["seq"] = s
    return c


def _np(t):
    return None if t is None else t.numpy()


def oracle_fwd(c, final=False):
    return oracle.fwd(_np(c["x"]), _np(c["w"]), _np(c["b"]), _np(c["seq"]), _np(c["init"]),
                      silu=c["silu"], final=final)


def oracle_bwd(c, need_dinit=None):
    if need_dinit is None:
        need_dinit = c["init"] is not None
    return oracle.bwd(_np(c["x"]), _np(c["w"]), _np(c["dout"]), _np(c["b"]), _np(c["seq"]),
                      _np(c["init"]), _np(c["dfinal"]), need_dinit=need_dinit, silu=c["silu"])


def _close(a, b, rtol, atol):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.shape != b.shape:
        return False, f"shape {a.shape} vs {b.shape}"
    if a.size == 0:
        return True, "empty"
    err = np.abs(a - b) - (atol + rtol * np.abs(b))
    i = int(np.argmax(err))
    ok = bool(err.flat[i] <= 0)
    return ok, f"worst excess {err.flat[i]:.3g} at {np.unravel_index(i, a.shape)}: {a.flat[i]} vs {b.flat[i]}"


def _d(t):
    return None if t is None else t.double()


def check_fwd_closed_form(c):
    """Forward and final states vs float64 grouped F.conv1d (no seq_idx)."""
    out, fin = oracle_fwd(c, final=True)
    ref, rfin = cf.conv1d_fwd(_d(c["x"]), _d(c["w"]), _d(c["b"]), _d(c["init"]), c["silu"])
    ok1, d1 = _close(out, ref.numpy(), 1e-5, 2e-5)
    ok2, d2 = _close(fin, rfin.numpy(), 0, 0)
    return ok1 and ok2, f"out: {d1}; final: {d2}"


def check_fwd_shifted(c):
    """Forward vs the float64 shifted-sum form with sequence masks."""
    out, _ = oracle_fwd(c)
    ref, _ = cf.shifted_fwd(_d(c["x"]), _d(c["w"]), _d(c["b"]), c["seq"], _d(c["init"]), c["silu"])
    return _close(out, ref.numpy(), 1e-5, 2e-5)


def check_bwd_autograd(c):
    """dx, dinit, dweight, dbias vs float64 autograd of the closed form (shifted form with seq)."""
    dx, dinit, dw, db = oracle_bwd(c)
    if c["seq"] is None:
        fn = cf.conv1d_fwd
        gx, gw, gb, gi = cf.autograd_bwd(fn, c["x"], c["w"], c["dout"], c["b"], c["init"],
                                         c["dfinal"], c["silu"])
    else:
        fn = cf.shifted_fwd
        gx, gw, gb, gi = cf.autograd_bwd(fn, c["x"], c["w"], c["dout"], c["b"], c["init"], None,
                                         c["silu"], seq=c["seq"])
    n = c["B"] * c["T"]
    res = [("dx", _close(dx, gx.numpy(), 1e-5, 5e-5))]
    res.append(("dweight", _close(dw, gw.numpy(), 1e-5, 1e-6 * n + 1e-5)))
    if c["b"] is not None:
        res.append(("dbias", _close(db, gb.numpy(), 1e-5, 1e-6 * n + 1e-5)))
    if c["init"] is not None:
        res.append(("dinit", _close(dinit, gi.numpy(), 1e-5, 5e-5)))
    ok = all(r[1][0] for r in res)
    return ok, "; ".join(f"{k}: {v[1]}" for k, v in res)


def check_brute(c):
    """Forward and backward vs the per-element definition (tiny shapes)."""
    L = lambda t: None if t is None else t.tolist()  # noqa: E731
    ref = cf.brute_fwd(L(c["x"]), L(c["w"]), L(c["b"]), L(c["seq"]), L(c["init"]), c["silu"])
    out, _ = oracle_fwd(c)
    ok1, d1 = _close(out, np.array(ref).reshape(out.shape), 1e-5, 2e-5)
    rdx, rdw, rdb, rdi = cf.brute_bwd(L(c["x"]), L(c["w"]), L(c["dout"]), L(c["b"]), L(c["seq"]),
                                      L(c["init"]), c["silu"], L(c["dfinal"]))
    dx, dinit, dw, db = oracle_bwd(c)
    res = [_close(dx, np.array(rdx).reshape(dx.shape), 1e-5, 5e-5),
           _close(dw, np.array(rdw), 1e-5, 1e-4)]
    if c["b"] is not None:
        res.append(_close(db, np.array(rdb), 1e-5, 1e-4))
    if c["init"] is not None:
        res.append(_close(dinit, np.array(rdi).reshape(dinit.shape), 1e-5, 5e-5))
    ok = ok1 and all(r[0] for r in res)
    return ok, d1 + " | " + " | ".join(r[1] for r in res)


def kat_cases():
    with open(_KAT) as f:
        return json.load(f)["cases"]


def check_kat(k):
    """Known-answer vectors (exact integers for the cases without activation)."""
    T = lambda v, dt=torch.float32: None if v is None else torch.tensor(v, dtype=dt)  # noqa: E731
    c = {"B": k["B"], "T": k["T"], "D": k["D"], "W": k["W"], "silu": k["silu"],
         "x": T(k["x"]), "w": T(k["weight"]), "b": T(k["bias"]), "init": T(k["initial_states"]),
         "seq": T(k["seq_idx"], torch.int32), "dout": T(k["dout"]), "dfinal": T(k["dfinal"])}
    rtol, atol = (0, 0) if k["exact"] else (1e-5, 1e-5)
    out, fin = oracle_fwd(c, final=k["seq_idx"] is None)
    res = [_close(out, np.array(k["out"], dtype=np.float64).reshape(out.shape), rtol, atol)]
    if fin is not None:
        res.append(_close(fin, np.array(k["final_states"]).reshape(fin.shape), 0, 0))
    dx, dinit, dw, db = oracle_bwd(c)
    res.append(_close(dx, np.array(k["dx"], dtype=np.float64).reshape(dx.shape), rtol, atol))
    res.append(_close(dw, np.array(k["dweight"], dtype=np.float64), rtol, atol))
    if k["dbias"] is not None:
        res.append(_close(db, np.array(k["dbias"], dtype=np.float64), rtol, atol))
    if k["dinit"] is not None:
        res.append(_close(dinit, np.array(k["dinit"], dtype=np.float64).reshape(dinit.shape),
                          rtol, atol))
    return all(r[0] for r in res), " | ".join(r[1] for r in res)


def check_seq_special(c):
    """Special cases of seq_idx that reduce to closed forms: all-equal ids equal the no-seq result
    bit for bit; all-distinct ids give act(w[P] x + b); padding rows give out == 0 and dx == 0."""
    res = []
    ce = dict(c, seq=torch.full((c["B"], c["T"]), 7, dtype=torch.int32), dfinal=None)
    cn = dict(c, seq=None, dfinal=None)
    oe, _ = oracle_fwd(ce)
    on, _ = oracle_fwd(cn)
    res.append(("equal-fwd", bool(np.array_equal(oe, on)), ""))
    dxe, _, dwe, _ = oracle_bwd(ce)
    dxn, _, dwn, _ = oracle_bwd(cn)
    res.append(("equal-dx", bool(np.array_equal(dxe, dxn)), ""))
    res.append(("equal-dw", bool(np.allclose(dwe, dwn, rtol=1e-12, atol=1e-12)), ""))
    B, T = c["B"], c["T"]
    cd = dict(c, seq=torch.arange(B * T, dtype=torch.int32).reshape(B, T) + 1, dfinal=None,
              init=None)
    od, _ = oracle_fwd(cd)
    P = c["W"] - 1
    z = c["w"][:, P].double() * c["x"].double()
    if c["b"] is not None:
        z = z + c["b"].double()
    ref = z * torch.sigmoid(z) if c["silu"] else z
    ok, det = _close(od, ref.numpy(), 1e-5, 2e-5)
    res.append(("distinct", ok, det))
    cp = dict(c, seq=torch.where(torch.arange(T) % 3 == 1, -1, 0).to(torch.int32).expand(B, T)
              .contiguous(), dfinal=None)
    op, _ = oracle_fwd(cp)
    dxp, _, _, _ = oracle_bwd(cp)
    pad = (cp["seq"] < 0).numpy()
    res.append(("pad-out", bool(np.all(op[pad] == 0)), ""))
    res.append(("pad-dx", bool(np.all(dxp[pad] == 0)), ""))
    return all(r[1] for r in res), "; ".join(f"{r[0]}={r[1]} {r[2]}" for r in res)


def check_state_handoff(c, split):
    """final_states == concat(init, x)[T-P:T] bit for bit, and a forward split at `split` with
    final_states passed on as initial_states equals the full forward bit for bit."""
    P = c["W"] - 1
    out, fin = oracle_fwd(c, final=True)
    pre = c["init"] if c["init"] is not None else torch.zeros(c["B"], P, c["D"])
    xx = torch.cat([pre, c["x"]], dim=1)
    ok1 = bool(np.array_equal(fin, xx[:, c["T"]:].numpy()))
    c1 = dict(c, x=c["x"][:, :split].contiguous(), T=split)
    o1, f1 = oracle_fwd(c1, final=True)
    c2 = dict(c, x=c["x"][:, split:].contiguous(), T=c["T"] - split, init=torch.from_numpy(f1))
    o2, f2 = oracle_fwd(c2, final=True)
    ok2 = bool(np.array_equal(np.concatenate([o1, o2], axis=1), out))
    ok3 = bool(np.array_equal(f2, fin))
    return ok1 and ok2 and ok3, f"final={ok1} chunked-out={ok2} chunked-final={ok3}"


def check_textbook_no_act(c):
    """Without activation: dbias = sum of dout, dweight[d, k] = sum_{b,t} dout * xx[t-P+k], and dx
    is the correlation of dout with the flipped kernel (plus dfinal on the last P rows)."""
    c = dict(c, silu=False, seq=None)
    dx, dinit, dw, db = oracle_bwd(c)
    B, T, D, W = c["B"], c["T"], c["D"], c["W"]
    P = W - 1
    dy = c["dout"].double()
    pre = c["init"].double() if c["init"] is not None else torch.zeros(B, P, D, dtype=torch.float64)
    xx = torch.cat([pre, c["x"].double()], dim=1)
    rdw = torch.stack([torch.einsum("btd,btd->d", dy, xx[:, k:k + T]) for k in range(W)], dim=1)
    res = [_close(dw, rdw.numpy(), 1e-6, 1e-6 * B * T + 1e-6)]
    if c["b"] is not None:
        res.append(_close(db, dy.sum(dim=(0, 1)).numpy(), 1e-6, 1e-6 * B * T + 1e-6))
    ypad = torch.cat([torch.zeros(B, P, D, dtype=torch.float64), dy,
                      torch.zeros(B, P, D, dtype=torch.float64)], dim=1)
    w = c["w"].double()
    rdxx = sum(w[:, P - j] * ypad[:, j:j + T + P] for j in range(W))  # rows -P .. T-1
    if c["dfinal"] is not None:
        rdxx[:, T:] += c["dfinal"].double()
    res.append(_close(dx, rdxx[:, P:].numpy(), 1e-5, 5e-5))
    if dinit is not None:
        res.append(_close(dinit, rdxx[:, :P].numpy(), 1e-5, 5e-5))
    return all(r[0] for r in res), " | ".join(r[1] for r in res)
