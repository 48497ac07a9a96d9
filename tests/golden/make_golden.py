#!/usr/bin/env python3
"""Writes tests/golden/gemm_golden.npz: small GEMM cases with their exact answers.

The fixtures pin the CPU oracle (oracle/ref_gemm.c) and the GPU path across
machines.  They are computed here WITHOUT the oracle:

* fp32, column-major (the hipBLAS view of test/test_gemm.c:32-58): inputs from
  glibc rand() through ctypes with test_gemm.c's formula
  (float)(rand() % 200 - 100) / 10 (test/test_gemm.c:70-73); the dot product
  is summed EXACTLY (fractions.Fraction) and rounded once to double, then
  C = alpha * (float)s + beta * C in float32, the expression of
  test/test_gemm.c:54.
* fp16, row-major engine contract (src/vkblas.h:21-26, test/test_h.c:63-79):
  inputs are numpy float16 of seeded normals; the exact dot product is rounded
  to double, then float32 alpha * (float)s + beta * old, then fp16 with
  round-to-nearest-even (numpy's float32 -> float16 cast).  An fp32-output
  variant (GemmEx 16F x 16F -> 32F) keeps the float32 value.
* closed forms: alpha = 0 (C = beta * C), K = 1 (outer product), an identity
  operand (exact copy), small integers (exact sums).

Shapes follow the fixture list planned for this path: 3x5x7, 33x65x17,
1x64x64 and 64x1x64, all four transpose variants.

  python tests/golden/make_golden.py      # rewrites gemm_golden.npz
"""
import ctypes
import json
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "gemm_golden.npz")
SHAPES = [(3, 5, 7), (33, 65, 17), (1, 64, 64), (64, 1, 64)]

_libc = ctypes.CDLL("libc.so.6")


def glibc_test_gemm_values(seed, n):
    _libc.srand(seed)
    return np.array([np.float32(_libc.rand() % 200 - 100) / np.float32(10.0) for _ in range(n)], np.float32)


def exact_dot(xs, ys):
    """Exact sum of float products, rounded once to double."""
    s = Fraction(0)
    for x, y in zip(xs, ys):
        s += Fraction(float(x)) * Fraction(float(y))
    return float(s)


def cm_case(ta, tb, m, n, k, alpha, beta, lda, ldb, ldc, seed):
    """hipBLAS column-major: C[i + j ldc] = alpha * sum_t op(A)[i,t] op(B)[t,j] + beta * C."""
    na = lda * (m if ta else k)
    nb = ldb * (k if tb else n)
    vals = glibc_test_gemm_values(seed, na + nb + ldc * n)
    A, B, C = vals[:na], vals[na:na + nb], vals[na + nb:]
    out = C.copy()
    for j in range(n):
        for i in range(m):
            a = [A[t + i * lda] if ta else A[i + t * lda] for t in range(k)]
            b = [B[j + t * ldb] if tb else B[t + j * ldb] for t in range(k)]
            s = np.float32(exact_dot(a, b))
            v = np.float32(alpha) * s
            if beta != 0.0:
                v = v + np.float32(beta) * C[i + j * ldc]
            out[i + j * ldc] = v
    return A, B, C, out


def rm_f16_case(op_a, op_b, M, N, K, alpha, beta, lda, ldb, ldc, seed):
    """Engine row-major contract, fp16 in; returns fp16 and fp32 results."""
    r = np.random.default_rng(seed)
    na = lda * (K if op_a else M)
    nb = ldb * (N if op_b else K)
    A = (r.standard_normal(na) / np.sqrt(K)).astype(np.float16)
    B = r.standard_normal(nb).astype(np.float16)
    C = r.standard_normal(ldc * M).astype(np.float16)
    Cf = C.astype(np.float32)
    out16, out32 = C.copy(), Cf.copy()
    for m in range(M):
        for n in range(N):
            a = [A[k * lda + m] if op_a else A[m * lda + k] for k in range(K)]
            b = [B[n * ldb + k] if op_b else B[k * ldb + n] for k in range(K)]
            s = np.float32(exact_dot([float(x) for x in a], [float(y) for y in b]))
            v16 = np.float32(alpha) * s
            v32 = np.float32(alpha) * s
            if beta != 0.0:
                v16 = v16 + np.float32(beta) * np.float32(C[m * ldc + n])
                v32 = v32 + np.float32(beta) * Cf[m * ldc + n]
            out16[m * ldc + n] = np.float16(v16)
            out32[m * ldc + n] = v32
    return A.view(np.uint16), B.view(np.uint16), C.view(np.uint16), Cf, out16.view(np.uint16), out32


def main():
    arrays, index = {}, []

    def add(name, meta, **arrs):
        index.append(dict(name=name, **meta))
        for k, v in arrs.items():
            arrays[f"{name}/{k}"] = v

    # fp32 column-major: tight ld, alpha 1, beta 0 (test_gemm.c's main list)
    for s, (m, n, k) in enumerate(SHAPES):
        for ta in (0, 1):
            for tb in (0, 1):
                lda = k if ta else m
                ldb = n if tb else k
                seed = 42 + 10 * s + 2 * ta + tb
                A, B, C, out = cm_case(ta, tb, m, n, k, 1.0, 0.0, lda, ldb, m, seed)
                add(f"f32cm_{m}x{n}x{k}_{'NT'[ta]}{'NT'[tb]}",
                    dict(kind="f32cm", ta=ta, tb=tb, m=m, n=n, k=k, alpha=1.0, beta=0.0, lda=lda, ldb=ldb, ldc=m),
                    A=A, B=B, C=C, out=out)
    # fp32 column-major: padded ld, alpha 0.5, beta 0.7
    for s, (m, n, k) in enumerate(SHAPES[:2]):
        for ta in (0, 1):
            for tb in (0, 1):
                lda = (k if ta else m) + 3
                ldb = (n if tb else k) + 2
                ldc = m + 5
                A, B, C, out = cm_case(ta, tb, m, n, k, 0.5, 0.7, lda, ldb, ldc, 1000 + 10 * s + 2 * ta + tb)
                add(f"f32cm_ab_{m}x{n}x{k}_{'NT'[ta]}{'NT'[tb]}",
                    dict(kind="f32cm", ta=ta, tb=tb, m=m, n=n, k=k, alpha=0.5, beta=0.7, lda=lda, ldb=ldb, ldc=ldc),
                    A=A, B=B, C=C, out=out)
    # fp16 row-major engine contract
    for s, (M, N, K) in enumerate(SHAPES):
        for op_a in (0, 1):
            for op_b in (0, 1):
                for alpha, beta in ((1.0, 0.0), (0.5, -0.25)):
                    lda = (M if op_a else K) + (1 if beta else 0)
                    ldb = (K if op_b else N) + (2 if beta else 0)
                    ldc = N + (3 if beta else 0)
                    tag = "" if beta == 0.0 else "ab_"
                    A, B, C, Cf, o16, o32 = rm_f16_case(op_a, op_b, M, N, K, alpha, beta, lda, ldb, ldc,
                                                        7000 + 100 * s + 10 * op_a + op_b + (5 if beta else 0))
                    add(f"f16rm_{tag}{M}x{N}x{K}_{op_a}{op_b}",
                        dict(kind="f16rm", op_a=op_a, op_b=op_b, M=M, N=N, K=K, alpha=alpha, beta=beta,
                             lda=lda, ldb=ldb, ldc=ldc),
                        A=A, B=B, C=C, Cf=Cf, out16=o16, out32=o32)
    # closed forms (fp32 column-major, values exact by construction)
    m, n, k = 33, 65, 17
    A, B, C = (glibc_test_gemm_values(s, c) for s, c in ((1, m * k), (2, k * n), (3, m * n)))
    add("closed_alpha0", dict(kind="f32cm", ta=0, tb=0, m=m, n=n, k=k, alpha=0.0, beta=0.7, lda=m, ldb=k, ldc=m),
        A=A, B=B, C=C, out=(np.float32(0.7) * C).astype(np.float32))
    a1, b1 = glibc_test_gemm_values(4, m), glibc_test_gemm_values(5, n)
    add("closed_outer_k1", dict(kind="f32cm", ta=0, tb=0, m=m, n=n, k=1, alpha=1.0, beta=0.0, lda=m, ldb=1, ldc=m),
        A=a1, B=b1, C=np.zeros(m * n, np.float32),
        out=(a1[:, None] * b1[None, :]).T.reshape(-1).astype(np.float32).copy())
    eye = np.eye(k, dtype=np.float32).reshape(-1)
    Bk = glibc_test_gemm_values(6, k * n)
    add("closed_identity", dict(kind="f32cm", ta=0, tb=0, m=k, n=n, k=k, alpha=1.0, beta=0.0, lda=k, ldb=k, ldc=k),
        A=eye, B=Bk, C=np.zeros(k * n, np.float32), out=Bk.copy())
    r = np.random.default_rng(99)
    Ai = r.integers(-8, 9, m * k).astype(np.float32)
    Bi = r.integers(-8, 9, k * n).astype(np.float32)
    Ci = np.zeros(m * n, np.float32)
    exact = (Ai.reshape(k, m).T.astype(np.int64) @ Bi.reshape(n, k).T.astype(np.int64)).T.reshape(-1)
    add("closed_integers", dict(kind="f32cm", ta=0, tb=0, m=m, n=n, k=k, alpha=1.0, beta=0.0, lda=m, ldb=k, ldc=m),
        A=Ai, B=Bi, C=Ci, out=exact.astype(np.float32))

    arrays["index"] = np.array(json.dumps(index))
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}: {len(index)} cases")


if __name__ == "__main__":
    main()
