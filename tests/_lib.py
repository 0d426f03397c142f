"""ctypes bindings used by the tests: the CPU oracle (oracle/liboracle.so, the checker) and the product library
(agens-engine_amd/libagens_kernels.so, called only through its C ABI).

bf16 tensors are numpy uint16 arrays of raw bit patterns, the int4 container is uint32.
"""
import ctypes
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
KERNELS_SO = os.path.join(ROOT, "agens-engine_amd", "libagens_kernels.so")
HEADER = os.path.join(ROOT, "include", "agens_kernels.h")

c_int, c_size_t, c_void_p, c_float, c_uint32, c_uint64 = (ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p,
                                                           ctypes.c_float, ctypes.c_uint32, ctypes.c_uint64)


def ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else ctypes.c_void_p(0)


# ------------------------------------------------------------------------------------------------ oracle
_ora = None


def oracle():
    """The CPU oracle (test infrastructure). Built by `make -C oracle` (also done by __graft_entry__.build())."""
    global _ora
    if _ora is None:
        if not os.path.exists(ORACLE_SO):
            import subprocess
            subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, capture_output=True)
        L = ctypes.CDLL(ORACLE_SO)
        V = None
        sigs = {
            "ora_bf2f": (c_float, [ctypes.c_uint16]),
            "ora_f2bf": (ctypes.c_uint16, [c_float]),
            "ora_pack_row": (c_int, [c_void_p, c_int, c_void_p]),
            "ora_unpack_row": (V, [c_void_p, c_int, c_void_p]),
            "ora_quantize_row": (V, [c_void_p, c_int, c_void_p, c_void_p]),
            "ora_kt_weight_bytes": (c_size_t, [c_int, c_int, c_int]),
            "ora_kt_scale_bytes": (c_size_t, [c_int, c_int, c_int]),
            "ora_repack_kt": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int]),
            "ora_kt_chunk": (V, [c_int, c_void_p, c_size_t, c_int, c_void_p]),
            "ora_dequant_kt_rows": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int]),
            "ora_gemv_ref_f32": (V, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                     c_int]),
            "ora_gemv_ref_f64": (V, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                     c_int]),
            "ora_gemv_exact_kt": (V, [c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                      c_int, c_int]),
            "ora_gemv_exact_kt_rows": (V, [c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                           c_int, c_int, c_int, c_int, c_int]),
            "ora_gemv_fast_kt": (V, [c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                     c_int]),
            "ora_gemv_fast_kt_rows": (V, [c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                          c_int, c_int, c_int]),
            "ora_fast_group_sum": (ctypes.c_longlong, [c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                                       ctypes.POINTER(c_int)]),
            "ora_xorshift32": (c_uint32, [ctypes.POINTER(c_uint32)]),
            "ora_hash_u32": (c_uint32, [c_uint64, c_uint64]),
            "ora_gen_container": (V, [c_uint64, c_int, c_int, c_int, c_int, c_void_p]),
            "ora_gen_scales": (V, [c_uint64, c_size_t, c_float, c_float, c_void_p]),
            "ora_gen_x": (V, [c_uint64, c_size_t, c_float, c_void_p]),
            "ora_i8_gemv": (V, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int]),
        }
        for name, (res, args) in sigs.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _ora = L
    return _ora


# host-side data helpers built on the oracle
def gen_container(seed, n, k, lo=-8, span=16):
    p = np.zeros(n * k // 8, dtype=np.uint32)
    oracle().ora_gen_container(seed, n, k, lo, span, ptr(p))
    return p


def gen_scales(seed, count, sa=0.02, sb=1e-4):
    s = np.zeros(count, dtype=np.uint16)
    oracle().ora_gen_scales(seed, count, sa, sb, ptr(s))
    return s


def gen_x(seed, count, xs=1.0):
    x = np.zeros(count, dtype=np.uint16)
    oracle().ora_gen_x(seed, count, xs, ptr(x))
    return x


class XorShift:
    """xorshift32 of the reference's gates (kernels/bench/test_w4.cu:36-40)."""

    def __init__(self, seed):
        self.s = c_uint32(seed)

    def __call__(self):
        return oracle().ora_xorshift32(ctypes.byref(self.s))

    def words(self, count):
        return np.array([self() for _ in range(count)], dtype=np.uint32)


def f2bf_array(f):
    """fp32 -> bf16 bits, round to nearest even (vectorised, finite values)."""
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf2f_array(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def ora_repack(bits, packed, scales, n, k, group):
    O = oracle()
    wt = np.zeros(O.ora_kt_weight_bytes(bits, n, k), dtype=np.uint8)
    st = np.zeros(O.ora_kt_scale_bytes(n, k, group) // 2, dtype=np.uint16)
    rc = O.ora_repack_kt(bits, ptr(packed), ptr(scales), ptr(wt), ptr(st), n, k, group)
    return rc, wt, st


def ora_fast(bits, x, m, wt, st, n, k, group, rows=None):
    y = np.zeros(m * n, dtype=np.uint16)
    r0, r1 = (0, n) if rows is None else rows
    oracle().ora_gemv_fast_kt_rows(bits, ptr(x), m, ptr(wt), ptr(st), ptr(y), n, n, k, group, r0, r1)
    return y.reshape(m, n)


def ora_exact(bits, x, m, wt, st, n, k, group, bf16w=0, rows=None):
    y = np.zeros(m * n, dtype=np.uint16)
    r0, r1 = (0, n) if rows is None else rows
    oracle().ora_gemv_exact_kt_rows(bits, ptr(x), m, ptr(wt), ptr(st), ptr(y), n, n, k, group, bf16w, r0, r1)
    return y.reshape(m, n)


def ora_ref_f32(x, m, packed, scales, n, k, group, nthreads=1):
    y = np.zeros(m * n, dtype=np.float32)
    oracle().ora_gemv_ref_f32(ptr(x), m, ptr(packed), ptr(scales), ptr(y), n, n, k, group, nthreads)
    return y.reshape(m, n)


def ora_ref_f64(x, m, packed, scales, n, k, group):
    y = np.zeros(m * n, dtype=np.float64)
    mag = np.zeros(m * n, dtype=np.float64)
    oracle().ora_gemv_ref_f64(ptr(x), m, ptr(packed), ptr(scales), ptr(y), ptr(mag), n, n, k, group)
    return y.reshape(m, n), mag.reshape(m, n)


def ulp_bf16(v):
    """1 bf16 ulp of |v| (kernels/bench/test_w4.cu:52-56)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    out = np.full(a.shape, 1e-30)
    nz = a >= 1e-30
    out[nz] = np.ldexp(1.0, (np.floor(np.log2(a[nz])) - 7).astype(np.int64))
    return out


def max_rel(y_bits, ref):
    """max |y - ref| / (|ref| + 1e-2): the error measure of kernels/bench/bench_gemv.cu:146-148."""
    y = bf2f_array(y_bits).astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(y - ref) / (np.abs(ref) + 1e-2)))


def max_rel_excess(y_bits, ref):
    """Error added beyond the mandatory bf16 output rounding, relative as in max_rel:
    max (|y - ref| - |bf16_rn(ref) - ref|) / (|ref| + 1e-2).  A bf16 output alone can be 2^-8 ~ 3.9e-3 away from the
    unrounded fp32 reference (max_rel), so the BASELINE tolerance (2e-3) is applied to this excess."""
    y = bf2f_array(y_bits).astype(np.float64)
    ref = np.asarray(ref, dtype=np.float32)
    r = np.abs(bf2f_array(f2bf_array(ref)).astype(np.float64) - ref.astype(np.float64))
    ref = ref.astype(np.float64)
    return float(np.max((np.abs(y - ref) - r) / (np.abs(ref) + 1e-2)))


def max_ulp_bound(y_bits, ref64, mag):
    """max |y - ref| / (1 bf16 ulp(ref) + 1e-6 sum|x*w|) (kernels/bench/test_w4.cu:123-141); <= 1 passes."""
    y = bf2f_array(y_bits).astype(np.float64)
    return float(np.max(np.abs(y - ref64) / (ulp_bf16(ref64) + 1e-6 * mag)))


# ------------------------------------------------------------------------------------------------ product library
def header_symbols():
    """Function names declared in include/*.h (the C ABI and its tuning entry points)."""
    inc = os.path.dirname(HEADER)
    txt = "".join(open(os.path.join(inc, f)).read() for f in sorted(os.listdir(inc)) if f.endswith(".h"))
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ak_\w+)\s*\(", txt)))


class WqStep(ctypes.Structure):
    """ak_wq_step of include/agens_kernels.h (one GEMV step of a chain)."""
    _fields_ = [("bits", c_int), ("m", c_int), ("nseg", c_int), ("k", c_int), ("group", c_int), ("bf16w", c_int),
                ("x", c_void_p), ("wt", c_void_p * 4), ("st", c_void_p * 4), ("y", c_void_p * 4), ("n", c_int * 4),
                ("ldy", c_int * 4), ("independent", c_int), ("act", c_int)]


def _addr(v):
    if isinstance(v, Dev):
        return v.p.value
    return v.value if isinstance(v, c_void_p) else v


def wq_step(bits, x, m, lins, ys, k, group=128, ldy=None, independent=0, bf16w=0, act=0):
    """A chain step over the Linear segments `lins` with outputs `ys` (Dev or addresses), x a Dev or an address."""
    st = WqStep()
    st.bits, st.m, st.nseg, st.k, st.group, st.bf16w = bits, m, len(lins), k, group, bf16w
    st.x = _addr(x)
    for i, (L, y) in enumerate(zip(lins, ys)):
        st.wt[i], st.st[i], st.y[i], st.n[i] = L.wt.p.value, L.st.p.value, _addr(y), L.n
        st.ldy[i] = ldy[i] if ldy else 0
    st.independent = independent
    st.act = act
    return st


class Chain:
    """ak_wq_chain_create / _run / _destroy over a list of WqStep."""

    def __init__(self, steps):
        K = kernels()
        self.steps = (WqStep * len(steps))(*steps)
        self.h = c_void_p()
        check(K.ak_wq_chain_create(self.steps, len(steps), ctypes.byref(self.h)), "ak_wq_chain_create")

    @property
    def chained(self):
        return kernels().ak_wq_chain_chained(self.h) == 1

    def run(self):
        check(kernels().ak_wq_chain_run(self.h, None), "ak_wq_chain_run")

    def __del__(self):
        try:
            if self.h:
                kernels().ak_wq_chain_destroy(self.h)
                self.h = None
        except Exception:
            pass


_ker = None


def kernels():
    """The C-ABI library. Raises if it has not been built (the HIP path never falls back)."""
    global _ker
    if _ker is None:
        if not os.path.exists(KERNELS_SO):
            raise RuntimeError(f"{KERNELS_SO} missing: run `python agens-engine_amd/build.py` first")
        L = ctypes.CDLL(KERNELS_SO)
        vp, i = c_void_p, c_int
        sigs = {
            "ak_device_count": (i, [ctypes.POINTER(c_int)]),
            "ak_set_device": (i, [i]),
            "ak_device_name": (i, [i, ctypes.c_char_p, i]),
            "ak_malloc": (i, [ctypes.POINTER(c_void_p), c_size_t]),
            "ak_free": (i, [vp]),
            "ak_memcpy_h2d": (i, [vp, vp, c_size_t]),
            "ak_memcpy_d2h": (i, [vp, vp, c_size_t]),
            "ak_synchronize": (i, []),
            "ak_mem_info": (i, [ctypes.POINTER(c_size_t), ctypes.POINTER(c_size_t)]),
            "ak_error_string": (ctypes.c_char_p, [i]),
            "ak_host_alloc": (i, [ctypes.POINTER(c_void_p), c_size_t]),
            "ak_host_free": (i, [vp]),
            "ak_w4_kt_weight_bytes": (c_size_t, [i, i]),
            "ak_w4_kt_scale_bytes": (c_size_t, [i, i, i]),
            "ak_w3_kt_weight_bytes": (c_size_t, [i, i]),
            "ak_wq_kt_weight_bytes": (c_size_t, [i, i, i]),
            "ak_w4g128_kt_weight_bytes": (c_size_t, [i, i]),
            "ak_w4g128_kt_scale_bytes": (c_size_t, [i, i]),
            "ak_w4_repack_kt": (i, [vp, vp, vp, vp, i, i, i, vp]),
            "ak_w3_repack_kt": (i, [vp, vp, vp, vp, i, i, i, vp]),
            "ak_wq_repack_kt": (i, [i, vp, vp, vp, vp, i, i, i, vp]),
            "ak_w4g128_repack_kt": (i, [vp, vp, vp, vp, i, i, vp]),
            "ak_wq_gemv_kt_multi": (i, [i, vp, i, i, vp, vp, vp, vp, vp, i, i, i, vp]),
            "ak_wq_gemv_kt_multi_noalloc": (i, [i, vp, i, i, vp, vp, vp, vp, vp, i, i, i, vp]),
            "ak_w4_gemv_kt": (i, [vp, vp, vp, vp, i, i, i, i, vp]),
            "ak_w4_gemv_kt_multi": (i, [vp, i, vp, vp, vp, vp, i, i, i, vp]),
            "ak_w4_gemv_kt_batched": (i, [vp, vp, vp, vp, i, i, i, i, i, vp]),
            "ak_w3_gemv_kt": (i, [vp, vp, vp, vp, i, i, i, vp]),
            "ak_w3_gemv_kt_multi": (i, [vp, i, vp, vp, vp, vp, i, i, vp]),
            "ak_w3_gemv_kt_batched": (i, [vp, vp, vp, vp, i, i, i, i, vp]),
            "ak_w4_mma_gemv": (i, [vp, vp, vp, vp, i, i, i, i, vp]),
            "ak_w4g128_gemv_kt_bf16": (i, [vp, vp, vp, vp, i, i, vp]),
            "ak_w4g128_gemv_bf16": (i, [vp, vp, vp, vp, i, i, vp]),
            "ak_w4g128_gemv_bf16_variant": (i, [i, vp, vp, vp, vp, i, i, vp]),
            "ak_w4g128_gemv_kt_variant": (i, [i, vp, vp, vp, vp, i, i, vp]),
            "ak_w4g128_gemv_kt_tune": (i, [i, i, i, i, vp, vp, vp, vp, i, i, vp]),
            "ak_wq_dequant_kt_rows": (i, [i, vp, vp, vp, i, i, i, i, i, vp]),
            "ak_w4_dequant_kt": (i, [vp, vp, vp, i, i, i, vp]),
            "ak_w4_dequant_kt_rows": (i, [vp, vp, vp, i, i, i, i, i, vp]),
            "ak_w3_dequant_kt_rows": (i, [vp, vp, vp, i, i, i, i, i, vp]),
            "ak_bf16_linear_f32reduce": (i, [vp, vp, vp, i, i, i, vp]),
            "ak_bf16_linear_f32reduce_ld": (i, [vp, vp, vp, i, i, i, i, vp]),
            "ak_i8_gemv": (i, [vp, vp, vp, vp, i, i, i, i, vp]),
            "ak_wq_gemm_kt": (i, [i, vp, i, vp, vp, vp, i, i, i, i, vp]),
            "ak_bf16_gemv_bi": (i, [vp, vp, vp, vp, i, i, i, vp]),
            "ak_silu_mul": (i, [vp, vp, i, i, vp]),
            "ak_wq_gemv_kt_silu": (i, [i, vp, i, vp, vp, vp, i, i, i, i, vp]),
            "ak_silu_mul_part": (i, [vp, vp, i, i, i, vp]),
            "ak_bf16_gemv_bi_ld": (i, [vp, vp, vp, vp, i, i, i, ctypes.c_long, vp]),
            "ak_wq_chain_create": (i, [ctypes.POINTER(WqStep), i, ctypes.POINTER(c_void_p)]),
            "ak_wq_chain_run": (i, [vp, vp]),
            "ak_wq_chain_chained": (i, [vp]),
            "ak_wq_chain_destroy": (i, [vp]),
            "ak_wq_chain_status": (i, []),
            "ak_w4_set_mma": (i, [i]),
            "ak_wq_set_mm_min": (i, [i]),
            "ak_w4_set_lean": (i, [i]),
            "ak_w4_set_tma": (i, [i]),
        }
        for name, (res, args) in sigs.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _ker = L
    return _ker


def check(rc, what="call"):
    if rc != 0:
        msg = kernels().ak_error_string(rc)
        raise RuntimeError(f"{what}: error {rc} ({msg.decode() if msg else '?'})")


class Dev:
    """A device buffer owned by the test (ak_malloc / ak_free)."""

    def __init__(self, nbytes):
        self.nbytes = max(int(nbytes), 1)
        p = c_void_p()
        check(kernels().ak_malloc(ctypes.byref(p), self.nbytes), "ak_malloc")
        self.p = p

    @classmethod
    def of(cls, arr):
        arr = np.ascontiguousarray(arr)
        d = cls(arr.nbytes)
        check(kernels().ak_memcpy_h2d(d.p, ptr(arr), arr.nbytes), "h2d")
        return d

    def get(self, dtype, count):
        out = np.zeros(count, dtype=dtype)
        check(kernels().ak_memcpy_d2h(ptr(out), self.p, out.nbytes), "d2h")
        return out

    def addr(self, byte_offset=0):
        return c_void_p(self.p.value + byte_offset)

    def free(self):
        if self.p:
            kernels().ak_free(self.p)
            self.p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def ptr_array(values):
    arr = (c_void_p * len(values))()
    for j, v in enumerate(values):
        arr[j] = v.value if isinstance(v, c_void_p) else v
    return arr


def int_array(values):
    return (c_int * len(values))(*values)


class Linear:
    """One quantized linear on the device: container (host + device) and its KT copy of `bits` bits."""

    def __init__(self, packed, scales, n, k, group, bits):
        K = kernels()
        self.n, self.k, self.group, self.bits = n, k, group, bits
        self.packed, self.scales = packed, scales
        self.P, self.S = Dev.of(packed), Dev.of(scales)
        self.wt = Dev(K.ak_wq_kt_weight_bytes(bits, n, k))
        self.st = Dev(K.ak_w4_kt_scale_bytes(n, k, group))
        self.rc = K.ak_wq_repack_kt(bits, self.P.p, self.S.p, self.wt.p, self.st.p, n, k, group, None)

    def host_kt(self):
        K = kernels()
        check(K.ak_synchronize())
        wt = self.wt.get(np.uint8, K.ak_wq_kt_weight_bytes(self.bits, self.n, self.k))
        st = self.st.get(np.uint16, K.ak_w4_kt_scale_bytes(self.n, self.k, self.group) // 2)
        return wt, st


def gemv(bits, x_dev, m, lins, k, group, bf16w=0, ldy=None, ys=None):
    """ak_wq_gemv_kt_multi over `lins` (segments); returns the output buffers."""
    K = kernels()
    ns = [L.n for L in lins]
    if ys is None:
        ys = [Dev(m * (ldy[i] if ldy else L.n) * 2) for i, L in enumerate(lins)]
    rc = K.ak_wq_gemv_kt_multi(bits, x_dev.p if isinstance(x_dev, Dev) else x_dev, m, len(lins),
                               ptr_array([L.wt.p for L in lins]), ptr_array([L.st.p for L in lins]),
                               ptr_array([y.p if isinstance(y, Dev) else y for y in ys]), int_array(ns),
                               int_array(ldy) if ldy else None, k, group, bf16w, None)
    check(rc, "ak_wq_gemv_kt_multi")
    return ys
