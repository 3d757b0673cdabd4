// devprobe — what one MI355X (gfx950) sustains for the building blocks of the
// int8 GEMM main loop, measured with HIP events over whole-chip launches:
//
//  1. v_mfma_i32_32x32x32_i8 issue rate with operands held in registers
//     (low-entropy operands), 1, 2 and 4 waves per SIMD;
//  2. the same MFMAs fed by ds_read_b128 fragment reads with a workgroup
//     barrier every two k-steps, operands of low entropy vs uniformly random
//     bytes (the matrix cores' power, and so the clock, depends on the data);
//  3. (2) plus global_load_lds_dwordx4 traffic of the int8 GEMM's volume
//     (16 KiB per k-step per CU);
//  4. global -> LDS and global -> VGPR load rates per CU from a window that
//     stays in L2 and from one that does not.
//
// Every access is in bounds by construction (power-of-two windows, masks);
// every loop has a fixed trip count.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

#define CHK(x)                                                                     \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);   \
      return 1;                                                                    \
    }                                                                              \
  } while (0)

constexpr double kPeakInt8 = 5.0e15;  // dense int8 MFMA, ops/s
constexpr double kClock = 2.4e9;
constexpr int kCUs = 256;

__device__ __forceinline__ void dma16(const void* src, void* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
#endif
}

// 1. MFMAs on register operands, 4 independent accumulators per wave.
__global__ __launch_bounds__(256) void mfma_regs(int iters, int* out) {
  v16i acc[4];
  for (int i = 0; i < 4; i++) acc[i] = v16i{};
  const v4i a = {(int)threadIdx.x, 3, 5, 7}, b = {1, (int)blockIdx.x, 2, 9};
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[i], 0, 0, 0);
  }
  int s = 0;
  for (int i = 0; i < 4; i++)
    for (int r = 0; r < 16; r++) s += acc[i][r];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// 2./3. A 128x128 (4x4 MFMA tiles) wave tile per k-step: 8 fragment reads for
// the next k-step interleaved with the 16 MFMAs, a barrier every second
// k-step, and (DMA) 4 global_load_lds_dwordx4 per k-step per lane.
template <int RND, int DMA>
__global__ __launch_bounds__(256, 1) void mfma_lds(int iters, const uint8_t* src, int* out) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[65536 + 16384];
  for (int i = threadIdx.x; i < 65536 / 16; i += 256) {
    v4i v;
    if (RND) {
      unsigned h = i * 2654435761u + 12345u;
      for (int e = 0; e < 4; e++) {
        h ^= h << 13;
        h ^= h >> 17;
        h ^= h << 5;
        v[e] = (int)h;
      }
    } else {
      v = v4i{i, i * 3, i * 5, i * 7};
    }
    reinterpret_cast<v4i*>(lds)[i] = v;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  v16i acc[4][4];
  for (int i = 0; i < 4; i++)
    for (int j = 0; j < 4; j++) acc[i][j] = v16i{};
  v4i f[2][8];
  for (int i = 0; i < 8; i++) f[0][i] = f[1][i] = v4i{lane, i, wave, 1};
  const int base = lane * 16 + wave * 4096;
  // this wave's own 64 KiB window of a 16 MiB buffer
  const uint8_t* g = src + (((size_t)blockIdx.x * 4 + wave) * 65536) % (16u << 20) + lane * 16;
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int s = 0; s < 2; s++) {
      v4i(&cur)[8] = f[s];
      v4i(&nxt)[8] = f[s ^ 1];
      if (DMA) {
        __builtin_amdgcn_s_waitcnt(4 | (0x7 << 4) | (0xF << 8));  // vmcnt(4)
#pragma unroll
        for (int l = 0; l < 4; l++)
          dma16(g + ((((it * 2 + s) * 4 + l) * 1024) & 65535), lds + 65536 + (wave * 4 + l) * 1024);
      }
#pragma unroll
      for (int r = 0; r < 8; r++)
        nxt[r] = *reinterpret_cast<const v4i*>(lds + ((base + r * 1024 + s * 8192 + (it & 7) * 16384) & 65535));
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur[i], cur[4 + j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int q = 0; q < 8; q++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if (DMA) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
      }
      __builtin_amdgcn_sched_group_barrier(0x008, DMA ? 4 : 8, 0);
      if (s == 1) {
        __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x3 << 14));  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int s = lds[65536 + threadIdx.x];
  for (int i = 0; i < 4; i++)
    for (int j = 0; j < 4; j++)
      for (int r = 0; r < 16; r++) s += acc[i][j][r];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// 4. Load rates: each wave streams its own region of a power-of-two window,
// DEPTH KiB per step, waiting until at most one step is outstanding.
template <int DEPTH>
__global__ __launch_bounds__(256) void load_lds(const uint8_t* src, unsigned mask, int iters, int* out) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[4 * DEPTH * 1024];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  unsigned off = ((blockIdx.x * 4 + wave) * 8192u) & mask;
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int u = 0; u < DEPTH; u++)
      dma16(src + ((off + u * 1024u) & mask) + lane * 16, lds + (wave * DEPTH + u) * 1024);
    off = (off + DEPTH * 1024u * 131u) & mask;
    __builtin_amdgcn_s_waitcnt((DEPTH & 0xF) | (0x7 << 4) | (0xF << 8) | (((DEPTH >> 4) & 3) << 14));
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  out[blockIdx.x * 256 + threadIdx.x] = lds[threadIdx.x * 16];
}
template <int DEPTH>
__global__ __launch_bounds__(256) void load_vgpr(const uint8_t* src, unsigned mask, int iters, int* out) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  unsigned off = ((blockIdx.x * 4 + wave) * 8192u) & mask;
  v4i x = {0, 0, 0, 0};
  for (int it = 0; it < iters; it++) {
    v4i t[DEPTH];
#pragma unroll
    for (int u = 0; u < DEPTH; u++) t[u] = *reinterpret_cast<const v4i*>(src + ((off + u * 1024u) & mask) + lane * 16);
#pragma unroll
    for (int u = 0; u < DEPTH; u++) x ^= t[u];
    off = (off + DEPTH * 1024u * 131u) & mask;
  }
  out[blockIdx.x * 256 + threadIdx.x] = x[0] + x[1] + x[2] + x[3];
}

template <class F>
static float best_ms(F f) {
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return -1.0f;
  f();
  (void)hipDeviceSynchronize();
  float best = 1e30f;
  for (int r = 0; r < 5; r++) {
    (void)hipEventRecord(a);
    f();
    (void)hipEventRecord(b);
    (void)hipEventSynchronize(b);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, a, b);
    best = std::min(best, ms);
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return best;
}

int main() {
  hipDeviceProp_t prop;
  CHK(hipGetDeviceProperties(&prop, 0));
  std::printf("device %s, %d CUs; fractions are of %.1f POP/s dense int8, B/clk at %.1f GHz\n",
              prop.gcnArchName, prop.multiProcessorCount, kPeakInt8 / 1e15, kClock / 1e9);
  int* out;
  uint8_t* src;
  const size_t big = (size_t)1 << 30;
  CHK(hipMalloc(&out, 1024 * 256 * sizeof(int)));
  CHK(hipMalloc(&src, big));
  CHK(hipMemset(src, 1, big));

  std::printf("\n| probe | waves/SIMD | TOP/s | of peak |\n|---|---:|---:|---:|\n");
  for (int wps : {1, 2, 4}) {
    const int grid = kCUs * wps, iters = 4000;
    const float ms = best_ms([&] { mfma_regs<<<grid, 256>>>(iters, out); });
    const double ops = (double)grid * 4 * iters * 4 * 65536;
    std::printf("| 32x32x32 i8 MFMA, register operands | %d | %.0f | %.3f |\n", wps, ops / ms / 1e9,
                ops / ms / 1e-3 / kPeakInt8);
  }
  auto lds_probe = [&](const char* what, auto kern) {
    const int iters = 4000;
    const float ms = best_ms([&] { kern<<<kCUs, 256>>>(iters, src, out); });
    const double ops = (double)kCUs * 4 * iters * 2 * 16 * 65536;
    std::printf("| %s | 1 | %.0f | %.3f |\n", what, ops / ms / 1e9, ops / ms / 1e-3 / kPeakInt8);
  };
  lds_probe("+ 8 LDS fragment reads per 16 MFMAs, barrier per 2 k-steps, low-entropy bytes", mfma_lds<0, 0>);
  lds_probe("the same, uniformly random bytes", mfma_lds<1, 0>);
  lds_probe("the same + 16 KiB/k-step/CU global_load_lds, low-entropy bytes", mfma_lds<0, 1>);
  lds_probe("the same + 16 KiB/k-step/CU global_load_lds, random bytes", mfma_lds<1, 1>);

  std::printf("\n| load | window | waves/CU | KiB in flight per wave | TB/s | B/clk/CU |\n|---|---:|---:|---:|---:|---:|\n");
  for (size_t span : {(size_t)1 << 20, (size_t)64 << 20, big}) {
    for (int wpc : {4, 8, 16}) {
      const int grid = kCUs * wpc / 4, iters = 256;
      const unsigned mask = (unsigned)(span - 1);
      auto rep = [&](const char* what, int depth, float ms) {
        const double bytes = (double)grid * 4 * iters * depth * 1024;
        std::printf("| %s | %zu MiB | %d | %d | %.2f | %.1f |\n", what, span >> 20, wpc, depth,
                    bytes / ms / 1e9, bytes / (ms * 1e-3) / kCUs / kClock);
      };
      rep("global_load_lds_dwordx4", 8, best_ms([&] { load_lds<8><<<grid, 256>>>(src, mask, iters, out); }));
      rep("global_load_dwordx4", 8, best_ms([&] { load_vgpr<8><<<grid, 256>>>(src, mask, iters, out); }));
    }
  }
  CHK(hipFree(src));
  CHK(hipFree(out));
  return 0;
}
