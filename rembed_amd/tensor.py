"""Python mirror of rembed's internal/tensor GEMM family over the C ABI.

Names follow the reference (internal/tensor/pack.go, pack8.go,
pack_vnni.go): PackB / PackB8 / PackB8VNNI pack once and upload to HBM;
MatMulPacked / MatMulPacked8 / MatMulPackedVNNI run on device buffers.
Errors surface as RembedError carrying the RH_* code, where the reference
returns `error` (pack time) or panics (contract violations).
"""
import ctypes
import sys

import numpy as np

from . import _lib
from ._lib import check, lib


class Context:
    """One GPU and one HIP stream (rh_context)."""

    def __init__(self, device=0):
        h = ctypes.c_void_p()
        check(lib.rh_context_create(device, ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib.rh_context_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def sync(self):
        check(lib.rh_context_sync(self.h))

    @property
    def stream(self):
        return lib.rh_context_stream(self.h)

    def set_option(self, option, value):
        check(lib.rh_context_set_option(self.h, option, value))

    def set_f32_algo(self, algo):
        self.set_option(_lib.RH_CTX_F32_ALGO, algo)

    def set_bf_algo(self, algo):
        """0: weight-only int8 / fp32 GEMMs on pre-split bf16 planes; 1: the
        split inside the GEMM's main loop."""
        self.set_option(_lib.RH_CTX_BF_ALGO, algo)

    def alloc(self, nbytes):
        return DeviceBuffer(self, nbytes)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        buf = DeviceBuffer(self, arr.nbytes)
        if arr.nbytes:
            check(lib.rh_memcpy_h2d(self.h, buf.ptr, arr.ctypes.data, arr.nbytes))
        return buf

    def profile(self, on=True):
        check(lib.rh_profile_enable(self.h, 1 if on else 0))

    def profile_read(self, kind):
        st = _lib.ProfileStat()
        check(lib.rh_profile_read(self.h, kind, ctypes.byref(st)))
        return {"launches": st.launches, "total_ms": st.total_ms,
                "total_ops": st.total_ops, "total_bytes": st.total_bytes}


class DeviceBuffer:
    """Device memory from rh_malloc, freed with the object."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib.rh_malloc(ctx.h, max(self.nbytes, 1), ctypes.byref(p)))
        self.ptr = p.value

    def download(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            check(lib.rh_memcpy_d2h(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr and self.ctx.h:
            lib.rh_free(self.ctx.h, self.ptr)
        self.ptr = None

    def __del__(self):
        if sys.is_finalizing():
            return  # the HIP runtime may already be torn down
        try:
            self.free()
        except Exception:
            pass


class PackedWeight:
    """A dense weight quantized/packed once and resident in HBM (rh_weight)."""

    def __init__(self, ctx, mode, bT, k, n, bias=None):
        bT = np.ascontiguousarray(bT, dtype=np.float32)
        if bT.size != k * n:
            raise _lib.RembedError(_lib.RH_ERR_SHAPE,
                                   f"bT has {bT.size} floats, want {k * n}")
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        h = ctypes.c_void_p()
        check(lib.rh_pack_weight(ctx.h, mode, bT.ctypes.data,
                                 None if b is None else b.ctypes.data, k, n,
                                 ctypes.byref(h)))
        self.ctx, self.h, self.mode, self.K, self.N = ctx, h, mode, k, n

    def export(self):
        """Host copies: (q [n][k] int8 or None, scales [n] or None, colsum or None)."""
        q = sc = cs = None
        if self.mode != _lib.RH_MODE_F32:
            q = np.empty((self.N, self.K), np.int8)
            sc = np.empty(self.N, np.float32)
        if self.mode == _lib.RH_MODE_A8W8:
            cs = np.empty(self.N, np.int32)
        check(lib.rh_weight_export(self.h, None if q is None else q.ctypes.data,
                                   None if sc is None else sc.ctypes.data,
                                   None if cs is None else cs.ctypes.data))
        return q, sc, cs

    def close(self):
        if self.h:
            lib.rh_weight_destroy(self.h)
            self.h = None

    def __del__(self):
        if sys.is_finalizing():
            return  # the HIP runtime may already be torn down
        try:
            self.close()
        except Exception:
            pass


def PackB(ctx, bT, k, n, bias=None):
    """internal/tensor/pack.go:25 — fp32 weights."""
    return PackedWeight(ctx, _lib.RH_MODE_F32, bT, k, n, bias)


def PackB8(ctx, bT, k, n, bias=None):
    """internal/tensor/pack8.go:25 — weight-only int8, per-channel scales."""
    return PackedWeight(ctx, _lib.RH_MODE_W8, bT, k, n, bias)


def PackB8VNNI(ctx, bT, k, n, bias=None):
    """internal/tensor/pack_vnni.go:28 — int8 weights for u8 x s8 GEMM."""
    return PackedWeight(ctx, _lib.RH_MODE_A8W8, bT, k, n, bias)


class PackedGated(PackedWeight):
    """Gated-MLP weight: gate and up [i][k] packed interleaved
    (rh_pack_weight_gated); rh_linear with RH_ACT_SWIGLU / RH_ACT_GEGLU
    writes act(gate) * up, i columns. N is the packed row count 2i."""

    def __init__(self, ctx, mode, gate, up, k, i):
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        up = np.ascontiguousarray(up, dtype=np.float32)
        if gate.size != k * i or up.size != k * i:
            raise _lib.RembedError(_lib.RH_ERR_SHAPE, f"gate/up must be [{i}][{k}]")
        h = ctypes.c_void_p()
        check(lib.rh_pack_weight_gated(ctx.h, mode, gate.ctypes.data, up.ctypes.data, k, i,
                                       ctypes.byref(h)))
        self.ctx, self.h, self.mode, self.K, self.N = ctx, h, mode, k, 2 * i


def ldq_for(k):
    """Row stride of quantized activations: k rounded up to 16 bytes."""
    return (k + 15) // 16 * 16


def QuantizeRowsU8(ctx, a, m, k, qa, ldq, row_scales):
    """QuantizeRowU8 over m rows (pack_vnni.go:85-117), device buffers."""
    check(lib.rh_quantize_rows_u8(ctx.h, a.ptr, m, k, qa.ptr, ldq, row_scales.ptr))


def GELUQuantizeRowsU8(ctx, a, m, k, qa, ldq, row_scales):
    """GELU then QuantizeRowU8 (bert.go:910-916): the FFN1 -> FFN2 hand-over;
    k a multiple of 8, a left unmodified."""
    check(lib.rh_gelu_quantize_rows_u8(ctx.h, a.ptr, m, k, qa.ptr, ldq, row_scales.ptr))


def MatMul(ctx, dst, a, bT, m, k, n):
    """tensor.go:16-70 — dst[m][n] = a[m][k]·bTᵀ, raw fp32 weights (no pack)."""
    check(lib.rh_matmul(ctx.h, dst.ptr, a.ptr, bT.ptr, m, k, n))


def MatMulPacked(ctx, dst, a, pb, m):
    """pack.go:123 — dst[m][N] = a[m][K]·Wᵀ."""
    check(lib.rh_matmul_packed(ctx.h, dst.ptr, a.ptr, pb.h, m))


def MatMulPacked8(ctx, dst, a, pb, m):
    """pack8.go:80."""
    check(lib.rh_matmul_packed8(ctx.h, dst.ptr, a.ptr, pb.h, m))


def MatMulPackedVNNI(ctx, dst, a, pb, m, qa, ldq, row_scales):
    """pack_vnni.go:124 — quantizes a into qa/row_scales, then the u8·s8 GEMM."""
    check(lib.rh_matmul_packed_vnni(ctx.h, dst.ptr, a.ptr, pb.h, m, qa.ptr, ldq,
                                    row_scales.ptr))


def GemmU8S8I32(ctx, acc, qa, ldq, pb, m):
    """Raw VPDPBUSD-form int32 accumulators (vnni_amd64.s:22-82)."""
    check(lib.rh_gemm_u8s8_i32(ctx.h, acc.ptr, qa.ptr, ldq, pb.h, m))


def Attention(ctx, out, ldout, qkv, in_bf16, ldqkv, q_off, k_off, v_off, cu, batch, max_len,
              heads, kv_heads, dh, scale, causal=False, window=0, precision=1):
    """Softmax attention over a packed varlen batch (rh_attention): the
    per-text head loops of bert.go:853-902, qwen3.go:319-390, gemma3.go:318-356."""
    check(lib.rh_attention(ctx.h, qkv.ptr, int(in_bf16), ldqkv, q_off, k_off, v_off, cu.ptr,
                           batch, max_len, heads, kv_heads, dh, float(scale), int(causal),
                           window, precision, out.ptr, ldout))


def AttentionPlanes(ctx, out, ldout, hi, lo, ldqkv, q_off, k_off, v_off, cu, batch, max_len,
                    heads, kv_heads, dh, scale, causal=False, window=0):
    """fp32-grade attention on the q|k|v rows' bf16 hi/lo split (rh_attention_planes)."""
    check(lib.rh_attention_planes(ctx.h, hi.ptr, lo.ptr, ldqkv, q_off, k_off, v_off, cu.ptr,
                                  batch, max_len, heads, kv_heads, dh, float(scale),
                                  int(causal), window, out.ptr, ldout))


def Linear(ctx, dst, a, pb, m, act=_lib.RH_ACT_NONE, qa=None, ldq=0, row_scales=None):
    """applyDense with fused bias/activation (bert.go:282-301)."""
    check(lib.rh_linear(ctx.h, dst.ptr, a.ptr, pb.h, m, act,
                        None if qa is None else qa.ptr, ldq,
                        None if row_scales is None else row_scales.ptr))


def LinearNoAlloc(ctx, dst, a, pb, m, act=_lib.RH_ACT_NONE):
    """rh_linear without allocating: staging in the library's fixed device
    scratch (rh_linear_noalloc)."""
    check(lib.rh_linear_noalloc(ctx.h, dst.ptr, a.ptr, pb.h, m, act))


def LinearU8(ctx, qa, ldq, row_scales, pb, m, act, qa_out, ldq_out, rs_out, absmax):
    """applyDense + QuantizeRowU8 of the output rows (rh_linear_u8)."""
    check(lib.rh_linear_u8(ctx.h, qa.ptr, ldq, row_scales.ptr, pb.h, m, act, qa_out.ptr,
                           ldq_out, rs_out.ptr, absmax.ptr))


# ---- host-array conveniences used by tests and the bench -----------------------

def matmul_host(ctx, a, pb, act=None):
    """Run the weight's GEMM on a host fp32 [m][K] array; returns host results.

    For RH_MODE_A8W8 also returns the quantized activations and row scales.
    """
    a = np.ascontiguousarray(a, dtype=np.float32)
    m = a.shape[0]
    da = ctx.upload(a)
    dst = ctx.alloc(m * pb.N * 4)
    extra = None
    if pb.mode == _lib.RH_MODE_A8W8:
        ldq = ldq_for(pb.K)
        qa = ctx.alloc(max(m, 1) * ldq)
        rs = ctx.alloc(max(m, 1) * 4)
        if act is None:
            MatMulPackedVNNI(ctx, dst, da, pb, m, qa, ldq, rs)
        else:
            Linear(ctx, dst, da, pb, m, act, qa, ldq, rs)
        ctx.sync()
        extra = (qa.download(np.uint8, (m, ldq)), rs.download(np.float32, (m,)))
    else:
        if act is not None:
            Linear(ctx, dst, da, pb, m, act)
        elif pb.mode == _lib.RH_MODE_W8:
            MatMulPacked8(ctx, dst, da, pb, m)
        else:
            MatMulPacked(ctx, dst, da, pb, m)
        ctx.sync()
    out = dst.download(np.float32, (m, pb.N))
    return (out, extra) if extra is not None else out
