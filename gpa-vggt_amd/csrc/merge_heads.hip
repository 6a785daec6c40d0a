// Deterministic segmented mean / sum of token rows (the K/V merge).
//
// For every output slot s of batch b, with token list
//   tokens[offsets[b*S + s] .. offsets[b*S + s + 1])       (positions in [0, N))
// and every head h:
//   out[b, h, s, :] = reduce_{n in list} t[b, h, n, :]       reduce = sum or mean
// accumulated in fp32 in list order and rounded once to the output type.
//
// This is the merge of merging/merge.py:234-250 (`merge.heads`, and `merge`
// with H = 1): the reference gathers the kept tokens and scatter_reduce_s the
// merged source rows into their destination slot (include_self=True), with
// atomics whose summation order varies from run to run (and, for bf16 V,
// bf16 partial sums).  Here the caller lists every slot's tokens (the slot's
// own token first, then its merged sources) once per merge, and the sum runs
// in that fixed order in fp32, so the result is reproducible bit for bit.
// Optionally the slot sizes (list lengths, merging/merge.py:211-217) and
// their logs (the attention bias, vggt/layers/attention.py:250-260) are
// written too.
//
// HBM-bound gather: each slot's rows stream through 16-byte loads (four
// fp32 or eight 16-bit elements per thread per row), four rows in flight per
// thread; a head's 64-element row is one contiguous 256 / 128-byte segment.
#include "gpa_common.h"

#include <math.h>

namespace gpa {
namespace {

constexpr int kThreads = 256;

struct MergeArgs {
  const void* t;
  void* out;
  const int64_t* offsets;  // [B*S + 1]
  const int64_t* tokens;   // [B*N]
  float* size_out;         // [B*S] or null
  float* log_size_out;     // [B*S] or null
  int64_t B, H, N, S, D;
  int64_t t_sb, t_sh, t_sn, o_sb, o_sh, o_sn;
  int mean;
  int tps;  // threads per slot (power of two <= kThreads); kThreads / tps slots per workgroup
};

// 16 bytes of row elements as fp32: four fp32 or eight 16-bit values.
template <typename T>
struct Vec;
template <>
struct Vec<float> {
  static constexpr int kN = 4;
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = x[j];
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  }
};
template <>
struct Vec<__bf16> {
  static constexpr int kN = 8;
  static __device__ __forceinline__ void load(const __bf16* p, float (&v)[8]) {
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (float)x[j];
  }
  static __device__ __forceinline__ void store(__bf16* p, const float (&v)[8]) {
    bf16x8 x;
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (__bf16)v[j];
    *reinterpret_cast<bf16x8*>(p) = x;
  }
};
template <>
struct Vec<_Float16> {
  typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
  static constexpr int kN = 8;
  static __device__ __forceinline__ void load(const _Float16* p, float (&v)[8]) {
    const f16x8 x = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (float)x[j];
  }
  static __device__ __forceinline__ void store(_Float16* p, const float (&v)[8]) {
    f16x8 x;
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (_Float16)v[j];
    *reinterpret_cast<f16x8*>(p) = x;
  }
};

// Slots are spread over workgroups, kThreads / tps per workgroup; a slot's
// tps threads cover the H x D plane in 16-byte runs.  Token indices and list
// bounds come from device memory, so they are checked here: an entry
// outside [0, N) or a list outside [0, B*N] makes the slot NaN instead of
// reading out of bounds.  Four rows are loaded at a time; they are still
// added in list order.
template <typename T>
__global__ __launch_bounds__(kThreads) void merge_heads_kernel(MergeArgs a) {
  constexpr int V = Vec<T>::kN;
  const int tps = a.tps;
  const int64_t slot = (int64_t)blockIdx.x * (kThreads / tps) + threadIdx.x / tps;
  if (slot >= a.B * a.S) return;
  const int lt = threadIdx.x % tps;
  const int64_t b = slot / a.S, s = slot % a.S;
  int64_t beg = a.offsets[slot], end = a.offsets[slot + 1];
  const bool bad = beg < 0 || end < beg || end > a.B * a.N;
  if (bad) beg = end = 0;
  const int64_t count = end - beg;
  const T* tb = static_cast<const T*>(a.t) + b * a.t_sb;
  T* ob = static_cast<T*>(a.out) + b * a.o_sb + s * a.o_sn;
  const int64_t plane = a.H * a.D;
  const float scale = a.mean && count > 0 ? 1.0f / (float)count : 1.0f;

  for (int64_t e = (int64_t)lt * V; e < plane; e += (int64_t)tps * V) {
    const T* row = tb + (e / a.D) * a.t_sh + (e % a.D);
    float acc[V];
#pragma unroll
    for (int j = 0; j < V; ++j) acc[j] = 0.f;
    bool poison = bad;
    int64_t i = beg;
    for (; i + 4 <= end; i += 4) {
      float v[4][V];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t n = a.tokens[i + u];
        const bool ok = n >= 0 && n < a.N;
        poison = poison || !ok;
        Vec<T>::load(row + (ok ? n : 0) * a.t_sn, v[u]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < V; ++j) acc[j] += v[u][j];
    }
    for (; i < end; ++i) {
      const int64_t n = a.tokens[i];
      const bool ok = n >= 0 && n < a.N;
      poison = poison || !ok;
      float v[V];
      Vec<T>::load(row + (ok ? n : 0) * a.t_sn, v);
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] += v[j];
    }
#pragma unroll
    for (int j = 0; j < V; ++j) acc[j] = poison ? __builtin_nanf("") : acc[j] * scale;
    Vec<T>::store(ob + (e / a.D) * a.o_sh + (e % a.D), acc);
  }
  if (lt == 0) {
    if (a.size_out) a.size_out[slot] = bad ? __builtin_nanf("") : (float)count;
    if (a.log_size_out) a.log_size_out[slot] = bad ? __builtin_nanf("") : logf((float)count);
  }
}

}  // namespace
}  // namespace gpa

using namespace gpa;

extern "C" int gpa_merge_heads(const void* t, int dtype, void* out, const int64_t* offsets,
                               const int64_t* tokens, int64_t B, int64_t H, int64_t N, int64_t S,
                               int64_t D, int64_t t_sb, int64_t t_sh, int64_t t_sn, int64_t o_sb,
                               int64_t o_sh, int64_t o_sn, int mode, float* size_out,
                               float* log_size_out, void* stream) {
  gpa_clear_error();
  if (B < 0 || H < 0 || N < 0 || S < 0 || D < 0) {
    gpa_set_error("gpa_merge_heads: negative size");
    return GPA_E_INVALID;
  }
  if (B == 0 || S == 0) return GPA_OK;
  if (!offsets || (!tokens && N > 0) || ((!t || !out) && H * D > 0)) {
    gpa_set_error("gpa_merge_heads: null pointer");
    return GPA_E_INVALID;
  }
  if (mode != GPA_MERGE_SUM && mode != GPA_MERGE_MEAN) {
    gpa_set_error("gpa_merge_heads: unknown mode %d", mode);
    return GPA_E_INVALID;
  }
  int esize;
  switch (dtype) {
    case GPA_DTYPE_F32: esize = 4; break;
    case GPA_DTYPE_BF16:
    case GPA_DTYPE_F16: esize = 2; break;
    default:
      gpa_set_error("gpa_merge_heads: unknown dtype %d", dtype);
      return GPA_E_INVALID;
  }
  const int64_t vec = 16 / esize;  // elements per 16-byte access
  const int64_t align = 16;
  const bool aligned = D % vec == 0 && (uintptr_t)t % align == 0 && (uintptr_t)out % align == 0 &&
                       (t_sb * esize) % align == 0 && (t_sh * esize) % align == 0 &&
                       (t_sn * esize) % align == 0 && (o_sb * esize) % align == 0 &&
                       (o_sh * esize) % align == 0 && (o_sn * esize) % align == 0;
  if (!aligned) {
    gpa_set_error("gpa_merge_heads: rows must be 16-byte aligned with unit feature stride and D "
                  "a multiple of %lld",
                  (long long)vec);
    return GPA_E_INVALID;
  }
  if (B * S > 0x7fffffff) {
    gpa_set_error("gpa_merge_heads: B*S=%lld exceeds the grid limit", (long long)(B * S));
    return GPA_E_UNSUPPORTED;
  }
  MergeArgs a{};
  a.t = t;
  a.out = out;
  a.offsets = offsets;
  a.tokens = tokens;
  a.size_out = size_out;
  a.log_size_out = log_size_out;
  a.B = B; a.H = H; a.N = N; a.S = S; a.D = D;
  a.t_sb = t_sb; a.t_sh = t_sh; a.t_sn = t_sn;
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_sn = o_sn;
  a.mean = mode == GPA_MERGE_MEAN;
  int tps = 1;
  while (tps < kThreads && tps * vec < H * D) tps <<= 1;
  a.tps = tps;
  const int64_t per_wg = kThreads / tps;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((B * S + per_wg - 1) / per_wg)), block(kThreads);
  if (dtype == GPA_DTYPE_F32)
    hipLaunchKernelGGL(merge_heads_kernel<float>, grid, block, 0, s, a);
  else if (dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(merge_heads_kernel<__bf16>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(merge_heads_kernel<_Float16>, grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("gpa_merge_heads: launch failed: %s", hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}
