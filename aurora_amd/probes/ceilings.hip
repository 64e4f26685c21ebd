// Ceiling probes for the roofline figures the bench reports: what the GPU
// under test sustains for
//   * fp32 MFMA issue with every operand in registers (no memory traffic),
//   * a streaming read of a buffer far larger than the caches (the best of
//     a few load depths and grid sizes),
//   * an empty kernel replayed from a HIP graph (the fixed cost every
//     launch of the captured decode step pays),
//   * reads of a few MB replayed from a HIP graph, each launch reading its
//     own slice of a buffer larger than the last-level cache (cold: what a
//     decode-step kernel streaming one weight matrix once could cost) or all
//     the same slice (warm).
// A measurement aid built next to the library (libaurora_ceilings.so), not
// part of its C ABI.  All launches go to the caller's stream.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <type_traits>

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
constexpr int kChains = 8;  // independent accumulators per wave

// WIDE = false: v_mfma_f32_16x16x4_f32 (2048 FLOP, the form the GEMM and
// attention kernels use); true: v_mfma_f32_32x32x2_f32 (4096 FLOP).
template <bool WIDE>
__global__ void __launch_bounds__(256) mfma_f32_peak_kernel(int iters, float* sink) {
  using acc_t = typename std::conditional<WIDE, floatx16, floatx4>::type;
  constexpr int NE = WIDE ? 16 : 4;
  const float a = 1.0f + 1e-3f * (threadIdx.x & 7), b = 1.0f - 1e-3f * (threadIdx.x & 3);
  acc_t acc[kChains];
#pragma unroll
  for (int j = 0; j < kChains; ++j)
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[j][e] = 0.f;
  for (int i = 0; i < iters; ++i) {  // 4 rounds of the chains per trip
#pragma unroll
    for (int r = 0; r < 4 * kChains; ++r) {
      if constexpr (WIDE)
        acc[r % kChains] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[r % kChains], 0, 0, 0);
      else
        acc[r % kChains] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[r % kChains], 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kChains; ++j)
#pragma unroll
    for (int e = 0; e < NE; ++e) s += acc[j][e];
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Grid-stride read: lane i reads float4 i, i + S, i + 2S, … (S = all lanes
// of the grid), U loads in flight per lane per step.
template <int U, bool NT>
__global__ void __launch_bounds__(256) stream_read_kernel(const floatx4* __restrict__ src, size_t n4,
                                                          float* sink) {
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (U - 1) * stride < n4; i += U * stride) {
    floatx4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(src + i + u * stride) : src[i + u * stride];
#pragma unroll
    for (int u = 0; u < U; ++u) acc += v[u];
  }
  for (; i < n4; i += stride) acc += src[i];
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

__global__ void empty_kernel() {}

}  // namespace

extern "C" {

// FLOP of one ceil_mfma_f32 launch: blocks · 4 waves · iters · 4 · chains · 2·16·16·4.
double ceil_mfma_f32_flop(int blocks, int iters) {
  return (double)blocks * 4.0 * iters * 4 * kChains * 2048.0;
}

// sink: blocks · 256 floats of device memory.
int ceil_mfma_f32(void* stream, int blocks, int iters, float* sink) {
  if (blocks <= 0 || iters <= 0 || !sink) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_f32_peak_kernel<false>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, sink);
  return (int)hipGetLastError();
}

// The same probe with v_mfma_f32_32x32x2_f32: blocks · 4 · iters · 4 · chains · 2·32·32·2 FLOP.
double ceil_mfma_f32_32x32_flop(int blocks, int iters) {
  return (double)blocks * 4.0 * iters * 4 * kChains * 4096.0;
}

int ceil_mfma_f32_32x32(void* stream, int blocks, int iters, float* sink) {
  if (blocks <= 0 || iters <= 0 || !sink) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_f32_peak_kernel<true>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, sink);
  return (int)hipGetLastError();
}

// Reads `bytes` (a multiple of 16) at src once; sink: blocks · 256 floats.
// mode: 0 → 4 loads in flight per lane, 1 → 8, 2 → 8 non-temporal.
int ceil_stream_read(void* stream, const void* src, size_t bytes, int blocks, int mode, float* sink) {
  if (blocks <= 0 || !src || !sink || bytes % 16 != 0 || mode < 0 || mode > 2) return (int)hipErrorInvalidValue;
  const floatx4* s4 = static_cast<const floatx4*>(src);
  hipStream_t st = (hipStream_t)stream;
  if (mode == 0)
    hipLaunchKernelGGL((stream_read_kernel<4, false>), dim3(blocks), dim3(256), 0, st, s4, bytes / 16, sink);
  else if (mode == 1)
    hipLaunchKernelGGL((stream_read_kernel<8, false>), dim3(blocks), dim3(256), 0, st, s4, bytes / 16, sink);
  else
    hipLaunchKernelGGL((stream_read_kernel<8, true>), dim3(blocks), dim3(256), 0, st, s4, bytes / 16, sink);
  return (int)hipGetLastError();
}

// Captures `n` empty single-block launches on `stream` into a graph and
// instantiates it; ceil_graph_launch replays it, ceil_graph_destroy frees it.
int ceil_graph_create(void* stream, int n, void** exec) {
  if (n <= 0 || !exec) return (int)hipErrorInvalidValue;
  *exec = nullptr;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return (int)e;
  for (int i = 0; i < n; ++i) hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, st);
  hipGraph_t g = nullptr;
  e = hipStreamEndCapture(st, &g);
  if (e != hipSuccess) return (int)e;
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return (int)e;
  *exec = ex;
  return 0;
}

// Captures `n` dependent reads of `slice_bytes` each (a multiple of 16) on
// `stream` into a graph: launch i reads src + i·slice_bytes when cold != 0,
// else src every time.  blocks / mode as ceil_stream_read; the caller owns
// n·slice_bytes (cold) or slice_bytes (warm) at src.
int ceil_graph_reads_create(void* stream, const void* src, size_t slice_bytes, int n, int blocks, int mode,
                            int cold, float* sink, void** exec) {
  if (n <= 0 || !exec || blocks <= 0 || !src || !sink || slice_bytes % 16 != 0 || mode < 0 || mode > 2)
    return (int)hipErrorInvalidValue;
  *exec = nullptr;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return (int)e;
  for (int i = 0; i < n; ++i) {
    const char* p = static_cast<const char*>(src) + (cold ? (size_t)i * slice_bytes : 0);
    (void)ceil_stream_read(stream, p, slice_bytes, blocks, mode, sink);
  }
  hipGraph_t g = nullptr;
  e = hipStreamEndCapture(st, &g);
  if (e != hipSuccess) return (int)e;
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return (int)e;
  *exec = ex;
  return 0;
}

int ceil_graph_launch(void* stream, void* exec) {
  if (!exec) return (int)hipErrorInvalidValue;
  return (int)hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream);
}

int ceil_graph_destroy(void* exec) {
  if (!exec) return 0;
  return (int)hipGraphExecDestroy((hipGraphExec_t)exec);
}

}  // extern "C"
