// Internal definitions shared by the HIP translation units of libaurora_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/aurora_hip.h"

// The context: one device, one default-priority stream, and a grow-only
// workspace used by kernels that need scratch beyond the caller's tensors
// (split-K partial sums).  The workspace is allocated on first need and kept.
struct aur_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int cu_count = 0;
  std::string last_error;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  // This device's copy of the allocation-free entry point's scratch array
  // (its device address, from hipGetSymbolAddress at aur_init), or null with
  // the failing call's code in noalloc_err.
  float* noalloc_scratch = nullptr;
  int noalloc_err = 0;
};

namespace aur {

int set_error(aur_ctx* ctx, int code, const char* fmt, ...);

inline void bind_device(const aur_ctx* ctx) {
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != ctx->device) (void)hipSetDevice(ctx->device);
}

// Makes `ctx` own at least `bytes` of workspace; returns 0 or an error code.
int ensure_workspace(aur_ctx* ctx, size_t bytes);

// Looks up (once per device, with that device current) the device address of
// the allocation-free entry point's scratch array and stores it in ctx.
void noalloc_scratch_init(aur_ctx* ctx);

// Output forms fused into the GEMM store; v = (A·B)(row, col), and R, X, C2
// are addressed with C's leading dimension.
enum EpiMode : int {
  EPI_STORE = 0,     // C = v
  EPI_ACCUM = 1,     // C = C + v
  EPI_RESID = 2,     // C = R + v            (residual add)
  EPI_GELU = 3,      // C = v, C2 = gelu(v)  (FFN up-projection keeps both)
  EPI_GELU_BWD = 4,  // C = v · gelu'(X)     (FFN backward through the activation)
};

struct Epilogue {
  int mode = EPI_STORE;
  const float* R = nullptr;
  const float* X = nullptr;
  float* C2 = nullptr;
};

// Caller-owned scratch for split-K partial tiles (used instead of the
// context's grow-only workspace, e.g. by work captured into a HIP graph).
struct Workspace {
  float* ptr = nullptr;
  size_t floats = 0;
};

// C = epilogue(op(A)·op(B)).  a_kcontig: A(m,k) = A[m*lda+k], else A[k*lda+m];
// b_kcontig: B(k,n) = B[n*ldb+k], else B[k*ldb+n].  Enqueued on ctx's stream.
int gemm(aur_ctx* ctx, bool a_kcontig, bool b_kcontig, const float* A, int lda, const float* B,
         int ldb, float* C, int ldc, int M, int N, int K, const Epilogue& epi,
         const Workspace* ws = nullptr);
int gemm(aur_ctx* ctx, bool a_kcontig, bool b_kcontig, const float* A, int lda, const float* B,
         int ldb, float* C, int ldc, int M, int N, int K, bool accumulate);
// `batch` independent C = op(A)·op(B) (store), problem z at A + z·sA,
// B + z·sB, C + z·sC (strides in floats); one launch, no split-K.
int gemm_batched(aur_ctx* ctx, bool a_kcontig, bool b_kcontig, const float* A, int lda, long long sA,
                 const float* B, int ldb, long long sB, float* C, int ldc, long long sC, int M, int N, int K,
                 int batch);
// Decode-shaped A@Bᵀ (M ≤ 64) split into `splits` K ranges (each a multiple
// of 64 long, none empty) whose products are stored to P[splits][M][N] for
// the consumer to sum in range order.  gemm_nt_partials_splits gives the
// split count that keeps about one block per CU in flight.
int gemm_nt_partials_splits(int M, int N, int K);
int gemm_nt_partials(aur_ctx* ctx, const float* A, int lda, const float* B, int ldb, float* P, int M, int N,
                     int K, int splits);

}  // namespace aur

// Every entry point: a null context is refused, and the context's device is
// made current for the calling thread, so allocations and launches of one
// context go to its own GPU when a process drives several.
#define AUR_CHECK_CTX(ctx)                                   \
  do {                                                       \
    if ((ctx) == nullptr) return AUR_EINVAL;                 \
    aur::bind_device(ctx);                                   \
  } while (0)

// Records a failing HIP call in the context and returns its code.
#define AUR_HIP(ctx, expr)                                                     \
  do {                                                                         \
    hipError_t _e = (expr);                                                    \
    if (_e != hipSuccess)                                                      \
      return aur::set_error((ctx), (int)_e, "%s: %s", #expr,                   \
                            hipGetErrorString(_e));                            \
  } while (0)

// Checks the launch that was just enqueued.
#define AUR_LAUNCH_CHECK(ctx, name)                                            \
  do {                                                                         \
    hipError_t _e = hipGetLastError();                                         \
    if (_e != hipSuccess)                                                      \
      return aur::set_error((ctx), (int)_e, "launch %s: %s", (name),           \
                            hipGetErrorString(_e));                            \
  } while (0)

typedef float floatx4 __attribute__((ext_vector_type(4)));

// v_mfma_f32_16x16x4_f32: D(16x16) += A(16x4)·B(4x16) for one wave.
// Lane l supplies A[l%16][l/16] and B[l/16][l%16]; it receives
// D[4*(l/16)+i][l%16] in element i of the result.
__device__ __forceinline__ floatx4 mfma16x16x4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
