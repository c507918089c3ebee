"""Generates tests/golden/kat_exact.json: known-answer vectors for the causal depthwise conv1d, with
exact rational arithmetic, from the definition in the reference (README.md:7, :36-46;
causal_conv1d.py:1-9, :17-41, :129-138, :153-164, :274-321).

The formulation here is deliberately different from the oracle's loops: per batch row and channel,
the forward is a banded matrix A (T x (T+P)) applied to the padded column xx = concat(init|0, x),
with A[t, t+k] = w[k] * [s(t+k-P) == s(t)] and rows of padding positions zeroed; the backward is
dxx = A^T g (plus dfinal on the last P entries of xx), dweight[k] = sum_t g[t] xx[t+k] *
mask, dbias = sum_t g[t]. Inputs are small integers and there is no activation, so every value is an
exact integer (the silu case stores double-precision values computed from math.exp).

Run: python tests/golden/make_kat.py  (rewrites the fixture; needs only the standard library)
"""

import json
import math
import os
import random
from fractions import Fraction

_HERE = os.path.dirname(os.path.abspath(__file__))


def _case(name, B, T, D, W, bias, init, seq, dfinal, silu, seed):
    rnd = random.Random(seed)
    P = W - 1
    ri = lambda: rnd.randint(-3, 3)  # noqa: E731
    x = [[[ri() for _ in range(D)] for _ in range(T)] for _ in range(B)]
    w = [[ri() for _ in range(W)] for _ in range(D)]
    b = [ri() for _ in range(D)] if bias else None
    i0 = [[[ri() for _ in range(D)] for _ in range(P)] for _ in range(B)] if init else None
    dy = [[[ri() for _ in range(D)] for _ in range(T)] for _ in range(B)]
    df = [[[ri() for _ in range(D)] for _ in range(P)] for _ in range(B)] if dfinal else None
    sq = seq

    out = [[[None] * D for _ in range(T)] for _ in range(B)]
    fin = [[[None] * D for _ in range(P)] for _ in range(B)]
    dx = [[[None] * D for _ in range(T)] for _ in range(B)]
    dinit = [[[None] * D for _ in range(P)] for _ in range(B)]
    dw = [[Fraction(0)] * W for _ in range(D)]
    db = [Fraction(0)] * D
    for bb in range(B):
        # sequence id of padded position q (row q - P)
        def sid(q):
            r = q - P
            if sq is None:
                return 0
            if r >= T:
                return -1
            if r < 0:
                return sq[bb][0] if init else -1
            return sq[bb][r]

        for d in range(D):
            xx = [Fraction(i0[bb][q][d]) if init else Fraction(0) for q in range(P)]
            xx += [Fraction(x[bb][t][d]) for t in range(T)]
            mask = [[sid(t + k) == sid(t + P) for k in range(W)] for t in range(T)]
            A = [[Fraction(0)] * (T + P) for _ in range(T)]
            for t in range(T):
                pad = sq is not None and sid(t + P) < 0
                for k in range(W):
                    if not pad and mask[t][k]:
                        A[t][t + k] = Fraction(w[d][k])
            z = [sum(A[t][q] * xx[q] for q in range(T + P)) for t in range(T)]
            if bias:
                z = [z[t] + (0 if (sq is not None and sid(t + P) < 0) else b[d]) for t in range(T)]
            g = []
            for t in range(T):
                if silu:
                    zf = float(z[t])
                    s = 1.0 / (1.0 + math.exp(-zf))
                    out[bb][t][d] = zf * s
                    gt = dy[bb][t][d] * s * (1.0 + zf * (1.0 - s))
                    g.append(0.0 if (sq is not None and sid(t + P) < 0) else gt)
                else:
                    out[bb][t][d] = z[t]
                    g.append(Fraction(0) if (sq is not None and sid(t + P) < 0)
                             else Fraction(dy[bb][t][d]))
            for p in range(P):
                fin[bb][p][d] = xx[T + p]
            dxx = [sum(A[t][q] * g[t] for t in range(T)) for q in range(T + P)]
            if dfinal:
                for p in range(P):
                    dxx[T + p] += df[bb][p][d]
            for t in range(T):
                dx[bb][t][d] = dxx[t + P]
            for p in range(P):
                dinit[bb][p][d] = dxx[p]
            for t in range(T):
                for k in range(W):
                    if mask[t][k]:
                        dw[d][k] += g[t] * xx[t + k]
                db[d] += g[t]

    def num(v):
        if isinstance(v, Fraction):
            assert v.denominator == 1
            return int(v)
        return v

    def nested(a):
        if isinstance(a, list):
            return [nested(v) for v in a]
        return num(a)

    return {
        "name": name, "B": B, "T": T, "D": D, "W": W, "silu": silu, "exact": not silu,
        "x": x, "weight": w, "bias": b, "initial_states": i0, "seq_idx": sq, "dout": dy,
        "dfinal": df,
        "out": nested(out), "final_states": nested(fin) if sq is None else None,
        "dx": nested(dx), "dinit": nested(dinit) if init else None,
        "dweight": nested(dw), "dbias": nested(db) if bias else None,
    }


def main():
    cases = [
        _case("plain_w3", 1, 5, 2, 3, bias=False, init=False, seq=None, dfinal=False, silu=False,
              seed=1),
        _case("bias_init_w4", 2, 4, 3, 4, bias=True, init=True, seq=None, dfinal=True, silu=False,
              seed=2),
        _case("seq_init_w3", 1, 6, 2, 3, bias=True, init=True, seq=[[0, 0, 1, 1, -1, 1]],
              dfinal=False, silu=False, seed=3),
        _case("seq_nonmonotone_w4", 2, 7, 2, 4, bias=True, init=False,
              seq=[[2, 2, 0, 0, 0, 2, -3], [-1, 5, 5, 5, 1, 1, 1]], dfinal=False, silu=False,
              seed=4),
        _case("short_T_lt_P_w5", 1, 2, 2, 5, bias=True, init=True, seq=None, dfinal=True,
              silu=False, seed=5),
        _case("width2", 2, 3, 1, 2, bias=False, init=True, seq=None, dfinal=True, silu=False,
              seed=6),
        _case("silu_w4", 1, 6, 3, 4, bias=True, init=True, seq=None, dfinal=True, silu=True,
              seed=7),
    ]
    with open(os.path.join(_HERE, "kat_exact.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_kat.py", "cases": cases}, f, indent=None)
    print(f"wrote {len(cases)} cases")


if __name__ == "__main__":
    main()
