"""CPU checks of the C-ABI library: it loads, exports every function include/agens_kernels.h declares, and its host
logic (sizes, argument validation, switches) answers without a GPU."""
import ctypes

import pytest

from _lib import kernels, header_symbols, oracle, KERNELS_SO


@pytest.fixture(scope="module")
def K():
    import os
    if not os.path.exists(KERNELS_SO):
        import subprocess, sys
        subprocess.run([sys.executable, os.path.join(os.path.dirname(KERNELS_SO), "build.py")], check=True)
    return kernels()


def test_exports_every_declared_symbol(K):
    syms = header_symbols()
    assert len(syms) >= 40
    missing = [s for s in syms if not hasattr(K, s)]
    assert not missing, missing


def test_sizes_match_layout(K):
    O = oracle()
    for n, k in ((5120, 5120), (55296, 5120), (5120, 27648), (301, 1152), (77, 640)):
        for bits in (2, 3, 4):
            assert K.ak_wq_kt_weight_bytes(bits, n, k) == O.ora_kt_weight_bytes(bits, n, k)
        assert K.ak_w4_kt_weight_bytes(n, k) == O.ora_kt_weight_bytes(4, n, k)
        assert K.ak_w3_kt_weight_bytes(n, k) == O.ora_kt_weight_bytes(3, n, k)
        for g in (64, 128):
            assert K.ak_w4_kt_scale_bytes(n, k, g) == O.ora_kt_scale_bytes(n, k, g)
    # the fused gate+up W3 55296 x 5120 and the down W2 5120 x 27648 shapes (w4_gemv.cu:560-563, 821-822)
    assert K.ak_wq_kt_weight_bytes(3, 55296, 5120) == 106168320
    assert K.ak_w4_kt_scale_bytes(55296, 5120, 128) == 4423680
    assert K.ak_wq_kt_weight_bytes(2, 5120, 27648) == 35389440
    assert K.ak_w4_kt_scale_bytes(5120, 27648, 128) == 2211840


def test_invalid_arguments_return_1_without_a_gpu(K):
    # w4_gemv.cu:556, :714, :724, :855 (and :565 / :826 for repack): bad group / k / nseg / m / bits -> 1
    nul = ctypes.c_void_p(0)
    arr = (ctypes.c_void_p * 1)(1)
    n = (ctypes.c_int * 1)(16)
    assert K.ak_wq_gemv_kt_multi(4, arr[0], 1, 1, arr, arr, arr, n, None, 1024, 96, 0, None) == 1   # group
    assert K.ak_wq_gemv_kt_multi(4, arr[0], 1, 1, arr, arr, arr, n, None, 1000, 128, 0, None) == 1  # k % group
    assert K.ak_wq_gemv_kt_multi(4, arr[0], 1, 5, arr, arr, arr, n, None, 1024, 128, 0, None) == 1  # nseg
    assert K.ak_wq_gemv_kt_multi(4, arr[0], 0, 1, arr, arr, arr, n, None, 1024, 128, 0, None) == 1  # m
    assert K.ak_wq_gemv_kt_multi(4, arr[0], 129, 1, arr, arr, arr, n, None, 1024, 128, 0, None) == 1
    assert K.ak_wq_gemv_kt_multi(5, arr[0], 1, 1, arr, arr, arr, n, None, 1024, 128, 0, None) == 1  # bits
    assert K.ak_wq_repack_kt(5, nul, nul, nul, nul, 16, 1024, 128, None) == 1
    assert K.ak_w4_repack_kt(nul, nul, nul, nul, 16, 1000, 128, None) == 1
    assert K.ak_wq_dequant_kt_rows(4, nul, nul, nul, 16, 1024, 128, 10, 10, None) == 1  # r0 + nr > n
    assert K.ak_w4g128_gemv_kt_variant(33, nul, nul, nul, nul, 16, 1024, None) == 1
    assert K.ak_w4g128_gemv_kt_tune(3, 1, 8, 0, nul, nul, nul, nul, 16, 1024, None) == 1
    # i8_gemv.cu:74: m outside 1..16 or k % 16 -> 1
    one = ctypes.c_void_p(16)
    assert K.ak_i8_gemv(one, one, one, one, 0, 16, 1024, 16, None) == 1
    assert K.ak_i8_gemv(one, one, one, one, 17, 16, 1024, 16, None) == 1
    assert K.ak_i8_gemv(one, one, one, one, 1, 16, 1000, 16, None) == 1
    # bi_gemv.cu:276: m outside 1..128 or k % 32 -> 1
    assert K.ak_bf16_gemv_bi(one, one, None, one, 0, 16, 1024, None) == 1
    assert K.ak_bf16_gemv_bi(one, one, None, one, 129, 16, 1024, None) == 1
    assert K.ak_bf16_gemv_bi_ld(one, one, None, one, 1, 16, 1040, 16, None) == 1
    assert K.ak_bf16_gemv_bi_ld(one, one, None, one, 2, 16, 1024, 15, None) == 1  # ldy < n: token rows overlap
    # the fused prefill GEMM: bits, ldy < n, k % group, m < 1 -> 1 (before any device call)
    assert K.ak_wq_gemm_kt(5, one, 1, one, one, one, 16, 0, 1024, 128, None) == 1
    assert K.ak_wq_gemm_kt(4, one, 1, one, one, one, 16, 8, 1024, 128, None) == 1
    assert K.ak_wq_gemm_kt(4, one, 1, one, one, one, 16, 0, 1000, 128, None) == 1
    assert K.ak_wq_gemm_kt(4, one, 0, one, one, one, 16, 0, 1024, 128, None) == 1
    # the no-alloc GEMV refuses a call whose worst-case split-K scratch, 4096 + 64 * P * T * sum(ceil(n / 16)) bytes,
    # exceeds its 64 MiB static array (here 8 * 16 * 8750 blocks), before any device call
    ns = (ctypes.c_int * 1)(140000)
    assert K.ak_wq_gemv_kt_multi_noalloc(4, one, 16, 1, None, None, None, ns, None, 8192, 128, 0, None) == 1
    # silu_mul.cu:59 / :67: sizes not multiples of 8, a share past the row -> 1
    assert K.ak_silu_mul(one, one, 2, 100, None) == 1
    assert K.ak_silu_mul_part(one, one, 64, 4, 8, None) == 1
    assert K.ak_silu_mul_part(one, one, 64, 56, 16, None) == 1


def test_switches(K):
    assert K.ak_w4_set_mma(0) == 0 and K.ak_w4_set_mma(1) == 0 and K.ak_w4_set_mma(-1) == 0
    assert K.ak_w4_set_lean(2) == 0 and K.ak_w4_set_lean(-1) == 0
    assert K.ak_w4_set_tma(4) == 0 and K.ak_w4_set_tma(-1) == 0
    assert K.ak_error_string(1)


def test_chain_invalid_arguments_return_1_without_a_gpu(K):
    from _lib import WqStep
    h = ctypes.c_void_p()
    st = (WqStep * 1)()
    s = st[0]
    s.bits, s.m, s.nseg, s.k, s.group, s.x = 4, 1, 1, 1024, 128, 1
    s.wt[0] = s.st[0] = s.y[0] = 1
    s.n[0] = 16
    assert K.ak_wq_chain_create(st, 0, ctypes.byref(h)) == 1  # no steps
    assert K.ak_wq_chain_create(None, 1, ctypes.byref(h)) == 1
    for field, bad in (("group", 96), ("k", 1000), ("nseg", 5), ("m", 0), ("m", 129), ("bits", 5)):
        good = getattr(s, field)
        setattr(s, field, bad)
        assert K.ak_wq_chain_create(st, 1, ctypes.byref(h)) == 1, field
        setattr(s, field, good)
    s.ldy[0] = 8  # ldy below n
    assert K.ak_wq_chain_create(st, 1, ctypes.byref(h)) == 1
    assert K.ak_wq_chain_run(None, None) == 1
    assert K.ak_wq_chain_destroy(None) == 0


def test_launch_table_pins_are_honoured(K):
    """Every shape pinned in csrc/wq_launch_table.h (written by tune_launch.py from measurements) is launched with its
    pinned configuration (ak_wq_tune_query, no device needed), and the tuner's override takes precedence until
    cleared.  The bits do not depend on the configuration (the GPU parity tests and the tuner check that)."""
    import ctypes
    import os
    import re
    ci = ctypes.c_int
    K.ak_wq_tune_query.argtypes = [ci, ci, ci, ctypes.POINTER(ci), ci, ctypes.POINTER(ci), ctypes.POINTER(ci),
                                   ctypes.POINTER(ci)]
    K.ak_wq_tune_override.argtypes = [ci, ci, ci]
    tab = open(os.path.join(os.path.dirname(KERNELS_SO), "csrc", "wq_launch_table.h")).read()
    num = r"(-?\d+)"
    pins = re.findall(r"\{" + ", ".join([num] * 4) + r", \{" + ", ".join([num] * 4) + r"\}, " + ", ".join([num] * 4) + r"\}", tab)
    got = [ci(), ci(), ci()]
    for p in pins:
        bits, m, k, nseg, n0, n1, n2, n3, split, nwv, sk, csplit = (int(v) for v in p)
        if bits == 0:
            continue
        ns = (ci * 4)(n0, n1, n2, n3)
        assert K.ak_wq_tune_query(bits, m, nseg, ns, k, *[ctypes.byref(g) for g in got]) == 0
        want = (1, 16, 1) if sk == 1 else (split, nwv, 0)
        assert tuple(g.value for g in got) == want, (p, [g.value for g in got])
    # the override wins, and clearing it restores the plan
    ns = (ci * 4)(5120, 0, 0, 0)
    assert K.ak_wq_tune_query(3, 1, 1, ns, 5120, *[ctypes.byref(g) for g in got]) == 0
    before = tuple(g.value for g in got)
    K.ak_wq_tune_override(2, 8, 0)
    assert K.ak_wq_tune_query(3, 1, 1, ns, 5120, *[ctypes.byref(g) for g in got]) == 0
    assert tuple(g.value for g in got) == (2, 8, 0)
    K.ak_wq_tune_override(0, 0, -1)
    assert K.ak_wq_tune_query(3, 1, 1, ns, 5120, *[ctypes.byref(g) for g in got]) == 0
    assert tuple(g.value for g in got) == before
