"""Write the golden fixtures under tests/golden/ (small, fp64, pure Python).

The expected outputs here are computed by brute-force pure-Python loops in
double precision with a *different algorithm* from the oracle's, so that they
pin the oracle rather than restate it:

- RMSNorm: y = x / sqrt(fsum(x^2)/n + eps) * w           (rmsnorm/original.py:38,51-52)
- RMSNorm bf16: the same with fp32 operations emulated by explicit rounding
           and the two bf16 rounding points of original.py:51-52; and rows
           whose output flips if 1/sqrt is one fp32 ulp off (rmsnorm_inv)
- SANA:    the O(N^2) quadratic form
           out[n][r] = sum_m (q_n . k_m) v_m[r] / (sum_m q_n . k_m + eps),
           q, k after ReLU -- algebraically equal to the linear form of
           LiteLA.attn_matmul (SANA_LinearAttention/original.py:99-117) that
           the oracle restates.
- FA:      explicit row softmax, LSE = log sum exp, and the JVP written out as
           tP_ij = P_ij (tS_ij - sum_k P_ik tS_ik), tO = tP v + P tv
           (flash-attention-jvp-derivation.md, Eqs. 3-5), bottom-right causal
           mask, GQA head mapping h -> h // (Hq/Hkv), empty rows -> 0 / +inf.

Inputs are drawn from Python's `random` with fixed seeds and rounded to
bf16-representable values (8 significant bits) so the same fixture also
serves 16-bit kernels exactly.  Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import math
import random
import struct
from pathlib import Path

HERE = Path(__file__).resolve().parent


def bf16_round(x: float) -> float:
    """Round to the nearest value with 8 significant bits (bf16 mantissa), ties to even."""
    if x == 0.0 or not math.isfinite(x):
        return x
    m, e = math.frexp(x)  # x = m * 2^e, 0.5 <= |m| < 1
    scaled = m * 256.0
    r = round(scaled)  # Python rounds half to even
    return math.ldexp(r / 256.0, e)


def draw(rng, n, mean=0.0, std=1.0):
    return [bf16_round(rng.gauss(mean, std)) for _ in range(n)]


def rmsnorm_cases():
    cases = []
    for seed, (rows, dim, eps) in enumerate([(2, 8, 1e-6), (3, 5, 1e-6), (1, 64, 1e-5), (2, 3, 0.5)]):
        rng = random.Random(100 + seed)
        x = [draw(rng, dim) for _ in range(rows)]
        w = draw(rng, dim, 1.0, 0.1)
        y = []
        for row in x:
            inv = 1.0 / math.sqrt(math.fsum(v * v for v in row) / dim + eps)
            y.append([row[c] * inv * w[c] for c in range(dim)])
        cases.append(dict(rows=rows, dim=dim, eps=eps, x=x, w=w, y=y))
    return cases


def f32(x: float) -> float:
    """Round a double to the nearest fp32 value (ties to even)."""
    return struct.unpack("<f", struct.pack("<f", x))[0]


def rmsnorm_bf16_cases():
    """bf16 RMSNorm with both rounding points of rmsnorm/original.py:51-52.

    Each row is drawn so that its sum of squares is exact in fp32 and its
    length is a power of two; the mean, ``+ eps``, ``sqrt`` and ``1/`` are
    then single fp32 operations, evaluated here in double and rounded to fp32
    (correct for these operations, since 53 >= 2*24 + 2).  Then
    ``n = bf16(f32(x * inv))`` (first rounding) and
    ``y = bf16(f32(n * w))`` (second rounding).  ``y_single`` is the same
    computation with one rounding at the end, ``bf16(f32(f32(x * inv) * w))``;
    each case holds elements where the two differ, so a kernel or oracle that
    drops the first rounding fails the fixture.
    """
    cases = []
    for seed, (rows, dim, eps) in enumerate([(4, 8, 1e-6), (3, 16, 1e-6), (2, 64, 1e-5), (2, 32, 1e-6)]):
        rng = random.Random(400 + seed)
        x, y, y_single = [], [], []
        w = draw(rng, dim, 1.0, 0.1)
        while len(x) < rows:
            row = draw(rng, dim, 0.0, 1.0)
            ss = math.fsum(v * v for v in row)
            if f32(ss) != ss:
                continue  # keep rows whose fp32 sum of squares is exact in any order
            inv = f32(1.0 / f32(math.sqrt(f32(f32(ss / dim) + f32(eps)))))
            n = [bf16_round(f32(v * inv)) for v in row]
            x.append(row)
            y.append([bf16_round(f32(n[c] * w[c])) for c in range(dim)])
            y_single.append([bf16_round(f32(f32(row[c] * inv) * w[c])) for c in range(dim)])
        assert any(a != b for ra, rb in zip(y, y_single) for a, b in zip(ra, rb)), "no double-rounding case"
        cases.append(dict(rows=rows, dim=dim, eps=eps, x=x, w=w, y=y, y_single=y_single))
    return cases


def f32_step(x: float, ulps: int) -> float:
    """The fp32 value `ulps` representable steps away from the fp32 value x (x > 0)."""
    bits = struct.unpack("<I", struct.pack("<f", x))[0]
    return struct.unpack("<f", struct.pack("<I", bits + ulps))[0]


def rmsnorm_inv_cases():
    """Rows whose bf16 output changes if 1/sqrt(mean + eps) is one fp32 ulp off.

    The values are multiples of 1/16 with |x| <= 2.5, so the fp32 sum of squares
    is exact in any order and mean = ss/64 is exact; eps (an fp32 value) is
    tuned so that some x_j * inv lands next to a bf16 rounding midpoint, where
    a one-ulp change of inv in the recorded direction flips bf16(x_j * inv).
    inv = f32(1 / f32(sqrt(f32(mean + eps)))), correctly rounded as above.
    ``y_off`` is the output with inv moved one ulp in ``direction``: it differs
    from ``y``, so these rows pin a correctly rounded inverse square root.
    """
    rng = random.Random(500)
    dim = 64
    cases = []
    for direction in (1, -1) * 4:
        found = None
        while found is None:
            row = [rng.randint(-40, 40) / 16 for _ in range(dim)]
            mean = math.fsum(v * v for v in row) / dim
            w = [bf16_round(1.0 + rng.randint(-8, 8) / 64) for _ in range(dim)]
            for j in rng.sample(range(dim), dim):
                if row[j] == 0.0:
                    continue
                mant, ex = math.frexp(row[j] / math.sqrt(mean + 1e-2))
                mid = math.copysign((math.floor(abs(mant) * 256) + 0.5) / 256, mant) * 2.0 ** ex
                eps0 = (row[j] / mid) ** 2 - mean
                if eps0 <= 1e-3:
                    continue
                for d in range(-100, 101):
                    eps = f32_step(f32(eps0), d)
                    inv = f32(1.0 / f32(math.sqrt(f32(mean + eps))))
                    n = [bf16_round(f32(v * inv)) for v in row]
                    off = f32_step(inv, direction)
                    n_off = [bf16_round(f32(v * off)) for v in row]
                    if n != n_off:
                        y = [bf16_round(f32(n[c] * w[c])) for c in range(dim)]
                        y_off = [bf16_round(f32(n_off[c] * w[c])) for c in range(dim)]
                        found = dict(rows=1, dim=dim, eps=eps, direction=direction, x=[row], w=w, y=[y],
                                     y_off=[y_off])
                        break
                if found is not None:
                    break
        cases.append(found)
    return cases


def sana_cases():
    cases = []
    for seed, (B, N, H, D) in enumerate([(1, 5, 2, 4), (2, 7, 1, 3), (1, 1, 3, 2), (1, 9, 2, 8)]):
        rng = random.Random(200 + seed)
        C = H * D
        qkv = [[[draw(rng, C) for _ in range(3)] for _ in range(N)] for _ in range(B)]
        eps = 1e-15
        out = [[[0.0] * C for _ in range(N)] for _ in range(B)]
        for b in range(B):
            for h in range(H):
                sl = slice(h * D, (h + 1) * D)
                q = [[max(v, 0.0) for v in qkv[b][n][0][sl]] for n in range(N)]
                k = [[max(v, 0.0) for v in qkv[b][n][1][sl]] for n in range(N)]
                v = [qkv[b][n][2][sl] for n in range(N)]
                for n in range(N):
                    a = [math.fsum(q[n][c] * k[m][c] for c in range(D)) for m in range(N)]
                    den = math.fsum(a) + eps
                    for r in range(D):
                        out[b][n][h * D + r] = math.fsum(a[m] * v[m][r] for m in range(N)) / den
        cases.append(dict(B=B, N=N, H=H, D=D, eps=eps, qkv=qkv, out=out))
    return cases


def fa_case(B, Nq, Nk, Hq, Hkv, D, causal, scale, seed):
    rng = random.Random(seed)
    gen = lambda n, h: [[[draw(rng, D) for _ in range(h)] for _ in range(n)] for _ in range(B)]  # noqa: E731
    q, k, v = gen(Nq, Hq), gen(Nk, Hkv), gen(Nk, Hkv)
    tq, tk, tv = gen(Nq, Hq), gen(Nk, Hkv), gen(Nk, Hkv)
    gamma = D ** -0.5 if scale is None else scale
    grp = Hq // Hkv
    out = [[[[0.0] * D for _ in range(Hq)] for _ in range(Nq)] for _ in range(B)]
    tout = [[[[0.0] * D for _ in range(Hq)] for _ in range(Nq)] for _ in range(B)]
    lse = [[[0.0] * Nq for _ in range(Hq)] for _ in range(B)]
    dot = lambda a, b: math.fsum(x * y for x, y in zip(a, b))  # noqa: E731
    for b in range(B):
        for h in range(Hq):
            hk = h // grp
            for i in range(Nq):
                valid = [(not causal) or j <= i + Nk - Nq for j in range(Nk)]
                if not any(valid):
                    lse[b][h][i] = math.inf
                    continue
                s = [gamma * dot(q[b][i][h], k[b][j][hk]) for j in range(Nk)]
                ts = [gamma * (dot(tq[b][i][h], k[b][j][hk]) + dot(q[b][i][h], tk[b][j][hk])) for j in range(Nk)]
                m = max(s[j] for j in range(Nk) if valid[j])
                e = [math.exp(s[j] - m) if valid[j] else 0.0 for j in range(Nk)]
                z = math.fsum(e)
                p = [x / z for x in e]
                lse[b][h][i] = m + math.log(z)
                c = math.fsum(p[j] * ts[j] for j in range(Nk))
                tp = [p[j] * (ts[j] - c) for j in range(Nk)]
                for d in range(D):
                    out[b][i][h][d] = math.fsum(p[j] * v[b][j][hk][d] for j in range(Nk))
                    tout[b][i][h][d] = math.fsum(tp[j] * v[b][j][hk][d] + p[j] * tv[b][j][hk][d] for j in range(Nk))
    return dict(B=B, Nq=Nq, Nk=Nk, Hq=Hq, Hkv=Hkv, D=D, causal=causal, scale=scale,
                q=q, k=k, v=v, tq=tq, tk=tk, tv=tv, out=out, tout=tout, lse=lse)


def fa_cases():
    specs = [
        (1, 3, 4, 2, 1, 4, False, None),
        (1, 4, 4, 2, 2, 8, True, None),
        (2, 5, 3, 2, 1, 4, True, 0.3),    # Nq > Nk: rows 0-1 have no valid key
        (1, 2, 6, 3, 3, 4, False, 0.7),
        (1, 1, 1, 1, 1, 8, True, None),
    ]
    return [fa_case(*s, seed=300 + i) for i, s in enumerate(specs)]


def main():
    for name, fn in (("rmsnorm", rmsnorm_cases), ("rmsnorm_bf16", rmsnorm_bf16_cases),
                     ("rmsnorm_inv", rmsnorm_inv_cases), ("sana", sana_cases), ("fa", fa_cases)):
        path = HERE / f"{name}_golden.json"
        path.write_text(json.dumps(fn(), allow_nan=True))
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
