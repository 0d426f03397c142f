"""The prefill GEMM (ak_bf16_linear_f32reduce / _ld: y = x W^T, bf16 in and out, fp32 accumulation; the reference's
kernels/src/bf16_linear.cu:68-92) on the GPU, against fp64 products of the same bf16 values.  The accumulation order
is the GEMM library's, so the bar is a tolerance: |y - ref| <= 1 bf16 ulp(ref) + 1e-5 sum |x w| (kernels/bench/
test_w4.cu:123-141 uses the same form).  The dequantize + GEMM route of linear() above 128 tokens is tested by the host
program (tests/host/test_linear.cpp)."""
import ctypes

import numpy as np
import pytest

from _lib import kernels, check, Dev, gen_x, bf2f_array, ulp_bf16, f2bf_array

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    K = kernels()
    n = ctypes.c_int(0)
    assert K.ak_device_count(ctypes.byref(n)) == 0 and n.value >= 1, "no GPU visible"
    yield K


def ref64(x, w):
    xf, wf = bf2f_array(x).astype(np.float64), bf2f_array(w).astype(np.float64)
    return xf @ wf.T, np.abs(xf) @ np.abs(wf).T


@pytest.mark.parametrize("m,n,k", [(129, 160, 1024), (256, 512, 5120), (300, 77, 640)])
def test_bf16_linear_f32reduce(m, n, k):
    K = kernels()
    x = gen_x(11 + m, m * k).reshape(m, k)
    w = f2bf_array(bf2f_array(gen_x(13 + n, n * k)) * 0.05).reshape(n, k)
    X, W, Y = Dev.of(x), Dev.of(w), Dev(m * n * 2)
    check(K.ak_bf16_linear_f32reduce(X.p, W.p, Y.p, m, n, k, None), "gemm")
    check(K.ak_synchronize(), "sync")
    y = bf2f_array(Y.get(np.uint16, m * n)).reshape(m, n).astype(np.float64)
    ref, mag = ref64(x, w)
    assert np.all(np.abs(y - ref) <= ulp_bf16(ref) + 1e-5 * mag)


def test_bf16_linear_f32reduce_ld_writes_its_columns_only():
    K = kernels()
    m, n, k, ldy, c0 = 200, 96, 1024, 300, 64
    x = gen_x(21, m * k).reshape(m, k)
    w = f2bf_array(bf2f_array(gen_x(23, n * k)) * 0.05).reshape(n, k)
    X, W = Dev.of(x), Dev.of(w)
    sentinel = np.full(m * ldy, 0x7FC1, dtype=np.uint16)
    Y = Dev.of(sentinel)
    check(K.ak_bf16_linear_f32reduce_ld(X.p, W.p, Y.addr(c0 * 2), m, n, k, ldy, None), "gemm ld")
    check(K.ak_synchronize(), "sync")
    yb = Y.get(np.uint16, m * ldy).reshape(m, ldy)
    assert np.all(yb[:, :c0] == 0x7FC1) and np.all(yb[:, c0 + n:] == 0x7FC1)
    y = bf2f_array(yb[:, c0:c0 + n]).astype(np.float64)
    ref, mag = ref64(x, w)
    assert np.all(np.abs(y - ref) <= ulp_bf16(ref) + 1e-5 * mag)


def test_bf16_linear_invalid_arguments():
    K = kernels()
    d = Dev(1024)
    assert K.ak_bf16_linear_f32reduce(d.p, d.p, d.p, 0, 4, 4, None) == 1
    assert K.ak_bf16_linear_f32reduce_ld(d.p, d.p, d.p, 4, 8, 4, 7, None) == 1  # ldy < n
