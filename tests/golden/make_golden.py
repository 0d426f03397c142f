"""Writes the golden fixtures of tests/golden/ (test infrastructure).

Inputs come from the generators of the reference's own GPU tests, restated here: kernels/bench/test_w4.cu:36-40
(xorshift32, state 12345; container words = rnd(), scales bf16(0.001 + 0.02 u), x bf16(-1 + 2 u) with
u = (rnd() >> 8) / 2^24, :75-77) and kernels/bench/test_wq.cu:36-40, 75-90 (state 2463534242; codes
lo + rnd() % span with the extremes forced at word 0, scales bf16(0.002 + 0.03 u)).  The reference holds no golden
output files, so the outputs are the oracle's (oracle/agq_oracle.c): they freeze its results, and the tests check them
against the fp64 closed form and the reference's bound.  Shapes are the reference tests' ragged ones (n = 77;
k = 640 and 1152, the latter padded to 2048 in the KT layout).

Usage: python tests/golden/make_golden.py   (writes tests/golden/*.npz)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import _lib as L  # noqa: E402

M = 4


class Rnd:
    """xorshift32 (test_w4.cu:37-40, test_wq.cu:37-40)."""

    def __init__(self, state):
        self.s = state

    def __call__(self):
        s = self.s
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        self.s = s
        return s


def f2bf(f):
    return int(L.f2bf_array(np.float32(f)))


def gen_w4(rnd, n, k, g):
    """test_w4.cu:75-77 (one case's data, in the test's order)."""
    packed = np.array([rnd() for _ in range(n * k // 8)], dtype=np.uint32)
    scales = np.array([f2bf(np.float32(0.001) + np.float32(0.02) * np.float32(rnd() >> 8) / np.float32(16777216.0))
                       for _ in range(n * (k // g))], dtype=np.uint16)
    x = np.array([f2bf(np.float32(-1.0) + np.float32(2.0) * np.float32(rnd() >> 8) / np.float32(16777216.0))
                  for _ in range(M * k)], dtype=np.uint16)
    return packed, scales, x


def gen_wq(rnd, n, k, g, bits):
    """test_wq.cu:75-90 (make) then the activations of :170-171."""
    lo, span = -(1 << (bits - 1)), 1 << bits
    words = []
    for w in range(n * k // 8):
        v = 0
        for j in range(8):
            q = lo + rnd() % span
            if w == 0 and j == 0:
                q = lo
            if w == 0 and j == 1:
                q = lo + span - 1
            v |= (q + 8) << (4 * j)
        words.append(v)
    packed = np.array(words, dtype=np.uint32)
    scales = np.array([f2bf(np.float32(0.002) + np.float32(0.03) * np.float32(rnd() >> 8) / np.float32(16777216.0))
                       for _ in range(n * (k // g))], dtype=np.uint16)
    x = np.array([f2bf(np.float32(-1.0) + np.float32(2.0) * np.float32(rnd() >> 8) / np.float32(16777216.0))
                  for _ in range(M * k)], dtype=np.uint16)
    return packed, scales, x


CASES = {  # name: (generator, state, bits, n, k, group)
    "w4_n77_k640_g64": ("w4", 12345, 4, 77, 640, 64),
    "w3_n77_k1152_g128": ("wq", 2463534242, 3, 77, 1152, 128),
    "w2_n77_k1152_g128": ("wq", 2463534242, 2, 77, 1152, 128),
}


def inputs(name):
    gen, state, bits, n, k, g = CASES[name]
    rnd = Rnd(state)
    return gen_w4(rnd, n, k, g) if gen == "w4" else gen_wq(rnd, n, k, g, bits)


def outputs(name, packed, scales, x):
    _, _, bits, n, k, g = CASES[name]
    rc, wt, st = L.ora_repack(bits, packed, scales, n, k, g)
    assert rc == 0
    deq = np.zeros(8 * k, dtype=np.uint16)
    L.oracle().ora_dequant_kt_rows(bits, L.ptr(wt), L.ptr(st), L.ptr(deq), n, k, g, n - 8, 8)
    out = {"wt": wt, "st": st, "deq_last8": deq}
    for m in (1, M):
        xm = x[: m * k]
        out[f"y_exact_m{m}"] = L.ora_exact(bits, xm, m, wt, st, n, k, g).reshape(-1)
        out[f"y_default_m{m}"] = L.ora_fast(bits, xm, m, wt, st, n, k, g).reshape(-1)
    ref, mag = L.ora_ref_f64(x, M, packed, scales, n, k, g)
    out["ref64"], out["mag64"] = ref.reshape(-1), mag.reshape(-1)
    return out


def main():
    for name in CASES:
        packed, scales, x = inputs(name)
        out = outputs(name, packed, scales, x)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), packed=packed, scales=scales, x=x, **out)
        print("wrote", name)


if __name__ == "__main__":
    main()
