// Content-adaptive pooled summaries of the frame-special shared K/V set.
//
// For every (batch b, head h, frame s) group of the frame's patch keys
// x_p = k[b, h, s*P + pts + p, :] (p < grid*grid, head dim 64):
//   seeds   y_g = x at the stride-kp lattice patches (gy*kp, gx*kp)
//   assign  a_p = argmax_g bf16( bf16(x_p / max(|x_p|, 1e-6)) . bf16(y_g / max(|y_g|, 1e-6)) )
//           (fp32 dot products rounded to bf16, lowest g on ties)
//   size    n_g = #{p : a_p = g}
//   pooled  K_g = sum_{a_p = g} k_p / max(n_g, 1),  V_g likewise from v
// written as pk, pv [B, H, S*npool, 64] bf16 and size [B, H, S, npool] fp32.
//
// This is the `_pool` of vggt/layers/attention.py:113-140 under bf16
// autocast: the normalised keys and seeds enter the einsum (:130) in bf16,
// its scores come back in bf16, argmax takes the first maximum, and the
// sums run in fp32 (scatter_add_, :132-139) before the cast back.  The
// reference's torch path sums with atomics in a run-dependent order; here
// the sums are fp32 LDS atomics too (the group's rows into 64-float
// accumulators per seed), so the last bits of a mean can differ between
// runs exactly as the reference's do.
//
// One workgroup (4 waves) per group: the seeds go to LDS, each thread
// assigns rows (64 FMAs per seed, seeds read as LDS broadcasts), then every
// wave adds two rows at a time (lane = feature pair) into the accumulators.
// HBM-bound: K read twice (the second read hits L2), V once.
#include "gpa_common.h"

#include <math.h>

namespace gpa {
namespace {

constexpr int kPoolThreads = 256;
constexpr int kPoolD = 64;
constexpr int kMaxPool = 64;      // seeds per frame (kp >= 5 at grid 37)
constexpr int kMaxPatches = 4096;

struct PoolArgs {
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* pk;
  uint16_t* pv;
  float* size;
  int32_t* assign;   // nullable
  int64_t k_sb, k_sh, k_sn, v_sb, v_sh, v_sn;
  int H, S, P, pts, grid, kp, nh, npool;
};

__device__ __forceinline__ float bf16_round(float x) { return (float)(__bf16)x; }

__global__ __launch_bounds__(kPoolThreads) void pool_shared_kernel(PoolArgs a) {
  __shared__ float seed[kMaxPool][kPoolD];          // normalised, bf16-rounded
  __shared__ float acc_k[kMaxPool][kPoolD];
  __shared__ float acc_v[kMaxPool][kPoolD];
  __shared__ int count[kMaxPool];
  __shared__ uint8_t asg[kMaxPatches];

  const int tid = threadIdx.x;
  const int grp = blockIdx.x;                  // (b*H + h)*S + s
  const int s = grp % a.S;
  const int bh = grp / a.S;
  const int h = bh % a.H, b = bh / a.H;
  const int npatch = a.grid * a.grid;
  const uint16_t* K = a.k + b * a.k_sb + h * a.k_sh + ((int64_t)s * a.P + a.pts) * a.k_sn;
  const uint16_t* Vp = a.v + b * a.v_sb + h * a.v_sh + ((int64_t)s * a.P + a.pts) * a.v_sn;

  // Row p of K as 64 floats; returns |x|^2.
  auto load_row = [&](int p, float (&x)[kPoolD]) {
    const bf16x8* r = reinterpret_cast<const bf16x8*>(K + (int64_t)p * a.k_sn);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < kPoolD / 8; ++c) {
      const bf16x8 v8 = r[c];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[8 * c + e] = (float)v8[e];
        ss = __builtin_fmaf(x[8 * c + e], x[8 * c + e], ss);
      }
    }
    return ss;
  };

  for (int i = tid; i < a.npool * kPoolD; i += kPoolThreads) {
    (&acc_k[0][0])[i] = 0.f;
    (&acc_v[0][0])[i] = 0.f;
  }
  for (int g = tid; g < a.npool; g += kPoolThreads) count[g] = 0;
  // Seeds: one thread per seed.
  for (int g = tid; g < a.npool; g += kPoolThreads) {
    const int gy = g / a.nh, gx = g % a.nh;
    float x[kPoolD];
    const float inv = 1.0f / fmaxf(__builtin_sqrtf(load_row(gy * a.kp * a.grid + gx * a.kp, x)), 1e-6f);
#pragma unroll
    for (int d = 0; d < kPoolD; ++d) seed[g][d] = bf16_round(x[d] * inv);
  }
  __syncthreads();

  // Assignment: one thread per row.
  for (int p = tid; p < npatch; p += kPoolThreads) {
    float x[kPoolD];
    const float inv = 1.0f / fmaxf(__builtin_sqrtf(load_row(p, x)), 1e-6f);
#pragma unroll
    for (int d = 0; d < kPoolD; ++d) x[d] = bf16_round(x[d] * inv);
    float best = -INFINITY;
    int bg = 0;
    for (int g = 0; g < a.npool; ++g) {
      float dot = 0.f;
#pragma unroll
      for (int d = 0; d < kPoolD; ++d) dot = __builtin_fmaf(x[d], seed[g][d], dot);
      dot = bf16_round(dot);
      if (dot > best) {
        best = dot;
        bg = g;
      }
    }
    asg[p] = (uint8_t)bg;
    atomicAdd(&count[bg], 1);
    if (a.assign) a.assign[(int64_t)grp * npatch + p] = bg;
  }
  __syncthreads();

  // Sums: a wave adds two rows per step, lane = (row parity, feature pair).
  const int lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, fp = (lane & 31) * 2;
  for (int p = 2 * wave + half; p < npatch; p += 2 * (kPoolThreads / 64)) {
    const int g = asg[p];
    const bf16x2 kv = *reinterpret_cast<const bf16x2*>(K + (int64_t)p * a.k_sn + fp);
    const bf16x2 vv = *reinterpret_cast<const bf16x2*>(Vp + (int64_t)p * a.v_sn + fp);
    atomicAdd(&acc_k[g][fp], (float)kv[0]);
    atomicAdd(&acc_k[g][fp + 1], (float)kv[1]);
    atomicAdd(&acc_v[g][fp], (float)vv[0]);
    atomicAdd(&acc_v[g][fp + 1], (float)vv[1]);
  }
  __syncthreads();

  const int64_t out_row0 = ((int64_t)bh * a.S + s) * a.npool;   // row of [B, H, S*npool]
  for (int i = tid; i < a.npool * kPoolD; i += kPoolThreads) {
    const int g = i / kPoolD, d = i % kPoolD;
    const float n = (float)count[g];
    const float inv = 1.0f / fmaxf(n, 1.0f);
    const int64_t o = (out_row0 + g) * kPoolD + d;
    const __bf16 mk = (__bf16)(acc_k[g][d] * inv), mv = (__bf16)(acc_v[g][d] * inv);
    a.pk[o] = __builtin_bit_cast(uint16_t, mk);
    a.pv[o] = __builtin_bit_cast(uint16_t, mv);
    if (d == 0) a.size[out_row0 + g] = n;
  }
}

}  // namespace
}  // namespace gpa

using namespace gpa;

extern "C" int gpa_pool_shared_bf16(const void* k, const void* v, void* pooled_k, void* pooled_v,
                                    float* size, int32_t* assign, int64_t B, int64_t H,
                                    int64_t S, int64_t P, int64_t pts, int64_t grid, int64_t kp,
                                    int64_t D, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                                    int64_t v_sb, int64_t v_sh, int64_t v_sn, void* stream) {
  gpa_clear_error();
  if (B < 0 || H < 0 || S < 0 || P < 0 || pts < 0 || grid < 0 || kp <= 0) {
    gpa_set_error("gpa_pool_shared_bf16: negative size or kp <= 0");
    return GPA_E_INVALID;
  }
  if (D != kPoolD) {
    gpa_set_error("gpa_pool_shared_bf16: head dim %lld unsupported (64 only)", (long long)D);
    return GPA_E_UNSUPPORTED;
  }
  if (B == 0 || H == 0 || S == 0 || grid == 0) return GPA_OK;
  if (!k || !v || !pooled_k || !pooled_v || !size) {
    gpa_set_error("gpa_pool_shared_bf16: null pointer");
    return GPA_E_INVALID;
  }
  if (P < pts + grid * grid) {
    gpa_set_error("gpa_pool_shared_bf16: frame of %lld tokens cannot hold %lld specials and a "
                  "%lldx%lld patch grid", (long long)P, (long long)pts, (long long)grid,
                  (long long)grid);
    return GPA_E_INVALID;
  }
  const int64_t nh = (grid + kp - 1) / kp;
  if (nh * nh > kMaxPool || grid * grid > kMaxPatches) {
    gpa_set_error("gpa_pool_shared_bf16: %lld seeds / %lld patches exceed the kernel's 64 / 4096",
                  (long long)(nh * nh), (long long)(grid * grid));
    return GPA_E_UNSUPPORTED;
  }
  const bool aligned = (uintptr_t)k % 16 == 0 && (uintptr_t)v % 4 == 0 && (B == 1 || k_sb % 8 == 0) &&
                       (H == 1 || k_sh % 8 == 0) && k_sn % 8 == 0 && v_sb % 2 == 0 &&
                       v_sh % 2 == 0 && v_sn % 2 == 0 && k_sn >= D && v_sn >= D;
  if (!aligned) {
    gpa_set_error("gpa_pool_shared_bf16: k rows must be 16-byte and v rows 4-byte aligned, unit "
                  "feature stride");
    return GPA_E_INVALID;
  }
  const int64_t groups = B * H * S;
  if (groups > 0x7fffffff) {
    gpa_set_error("gpa_pool_shared_bf16: too many groups");
    return GPA_E_UNSUPPORTED;
  }
  PoolArgs a{};
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.pk = (uint16_t*)pooled_k;
  a.pv = (uint16_t*)pooled_v;
  a.size = size;
  a.assign = assign;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_sn = k_sn;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_sn = v_sn;
  a.H = (int)H; a.S = (int)S; a.P = (int)P; a.pts = (int)pts; a.grid = (int)grid;
  a.kp = (int)kp; a.nh = (int)nh; a.npool = (int)(nh * nh);
  hipLaunchKernelGGL(pool_shared_kernel, dim3((unsigned)groups), dim3(kPoolThreads), 0,
                     (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("gpa_pool_shared_bf16: launch failed: %s", hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}
