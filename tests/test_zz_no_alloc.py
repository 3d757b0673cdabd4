"""rh_linear_noalloc against rh_linear, through the C ABI.

rh_linear_noalloc stages its intermediate data (full int8: u8 rows and row
scales; weight-only int8 / fp32: the bf16 planes of the activations) in the
library's fixed per-GPU device scratch instead of caller scratch or an
allocated workspace; it launches the same kernels, so its outputs must equal
rh_linear's bit for bit. Each case runs two calls in a row on the shared
scratch, the second with fewer rows, and checks a canary region past the
output. Sizes whose staging exceeds the scratch are refused before any
launch.
"""
import numpy as np
import pytest

from rembed_amd import _lib
from rembed_amd import tensor as T

pytestmark = pytest.mark.gpu

GUARD = 256  # canary floats past each output

CASES = [
    # mode, act, k, n (gated: n = i), gated
    (_lib.RH_MODE_A8W8, _lib.RH_ACT_NONE, 768, 768, False),
    (_lib.RH_MODE_A8W8, _lib.RH_ACT_GELU, 768, 3072, False),
    (_lib.RH_MODE_A8W8, _lib.RH_ACT_SWIGLU, 1024, 512, True),
    (_lib.RH_MODE_W8, _lib.RH_ACT_NONE, 1000, 1024, False),
    (_lib.RH_MODE_W8, _lib.RH_ACT_GEGLU, 768, 1152, True),
    (_lib.RH_MODE_F32, _lib.RH_ACT_GELU, 384, 1536, False),
    (_lib.RH_MODE_F32, _lib.RH_ACT_NONE, 3072, 768, False),
]
IDS = ["a8w8", "a8w8-gelu", "a8w8-swiglu", "w8-k1000", "w8-geglu", "f32-gelu", "f32-k3072"]


def run_pair(ctx, pw, a_host, n_out, act, bias_mode):
    m = a_host.shape[0]
    k = a_host.shape[1]
    a = ctx.upload(a_host)
    ref = ctx.upload(np.full(m * n_out + GUARD, 7.5, np.float32))
    got = ctx.upload(np.full(m * n_out + GUARD, 7.5, np.float32))
    if pw.mode == _lib.RH_MODE_A8W8:
        ldq = T.ldq_for(k)
        qa, rs = ctx.alloc(m * ldq), ctx.alloc(m * 4)
        T.Linear(ctx, ref, a, pw, m, act, qa, ldq, rs)
    else:
        T.Linear(ctx, ref, a, pw, m, act)
    T.LinearNoAlloc(ctx, got, a, pw, m, act)
    ctx.sync()
    r = ref.download(np.float32, (m * n_out + GUARD,))
    g = got.download(np.float32, (m * n_out + GUARD,))
    assert np.all(g[m * n_out:] == 7.5), "write past the output"
    assert np.array_equal(r[:m * n_out].view(np.uint32), g[:m * n_out].view(np.uint32))
    return g[:m * n_out]


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_noalloc_matches_rh_linear(gpu_ctx, case):
    mode, act, k, n, gated = case
    print(f"noalloc mode={mode} act={act} k={k} n={n} gated={gated}", flush=True)
    rng = np.random.default_rng(k + n + mode)
    if gated:
        gate = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        up = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        pw = T.PackedGated(gpu_ctx, mode, gate, up, k, n)
        n_out = n
    else:
        bT = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
        pw = T.PackedWeight(gpu_ctx, mode, bT, k, n, bias)
        n_out = n
    # two calls in a row on the shared scratch, the second smaller
    for m in (3001, 517):
        a_host = rng.standard_normal((m, k)).astype(np.float32)
        run_pair(gpu_ctx, pw, a_host, n_out, act, None)
    pw.close()


def test_noalloc_refuses_oversize_and_keeps_profiling(gpu_ctx):
    rng = np.random.default_rng(5)
    k, n = 3072, 64
    bT = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    pw = T.PackB8VNNI(gpu_ctx, bT, k, n)
    # full int8 stages m*3072 + 4m bytes: 21900 rows exceed 64 MiB
    m = 21900
    assert m * k + 4 * m > _lib.RH_NOALLOC_SCRATCH_BYTES
    a = gpu_ctx.upload(np.zeros((m, k), np.float32))
    dst = gpu_ctx.alloc(m * n * 4)
    with pytest.raises(_lib.RembedError) as e:
        T.LinearNoAlloc(gpu_ctx, dst, a, pw, m)
    assert e.value.code == _lib.RH_ERR_INVALID
    assert "scratch" in str(e.value)
    # the largest size that fits still runs, with event timing left on
    m2 = _lib.RH_NOALLOC_SCRATCH_BYTES // (k + 4) - 64
    a2 = rng.standard_normal((m2, k)).astype(np.float32)
    gpu_ctx.profile(True)
    try:
        g = run_pair(gpu_ctx, pw, a2, n, _lib.RH_ACT_NONE, None)
        st = gpu_ctx.profile_read(0)
        assert st["launches"] == 1  # only rh_linear's launch was timed
    finally:
        gpu_ctx.profile(False)
    assert np.all(np.isfinite(g))
    pw.close()
