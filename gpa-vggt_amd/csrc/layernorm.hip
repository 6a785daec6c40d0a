// Residual + LayerScale + LayerNorm of a pre-LN transformer block, fused,
// bf16 (or fp16) in and out, one wave per token row.
//
// For a row x (C features) and, optionally, a branch output y:
//   h   = bf16( x + bf16(gamma * y) )                  (y given)   else h = x
//   out = bf16( (h - mean(h)) * rsqrt(var(h) + eps) * w + b )   (fp32 math)
// where mean / var are the fp32 moments of the row (biased variance).
//
// This is the block step of vggt/layers/block.py:84-96 as it runs under
// bf16 autocast on a bf16 model: `x + self.ls1(attn_out)` multiplies and
// adds in bf16 (each op computed in fp32 and rounded), `self.norm2(h)` is
// on autocast's fp32 list (fp32 moments, fp32 output), and the next Linear
// casts that output to bf16.  The reference runs these as four to five
// passes over the [tokens, C] activations (mul, add, layer_norm, the
// autocast cast); here one read of x and y, and one write of h and out.
// Either output may be omitted: without y the kernel is the block's first
// LayerNorm; without an output it is the residual step alone.  The fp16
// instantiation is the same chain under fp16 autocast on an fp16 model (the
// reference's accuracy-evaluation stack): every bf16 rounding above becomes
// an fp16 rounding.
//
// Lane l of a row's wave owns features 8l + 512i .. +8 (i < C/512), so
// every load and store of the wave covers 1 KB of the row contiguously; the
// moments are wave reductions.  HBM-bound: 2 + 2 bytes read and 2 + 2
// written per feature when both outputs are asked for.
#include "gpa_common.h"

#include <math.h>

namespace gpa {
namespace {

constexpr int kRowsPerWG = 4;

struct LnArgs {
  const uint16_t* x;
  const uint16_t* y;      // nullable: no residual
  const uint16_t* gamma;  // [C], with y
  const uint16_t* w;      // [C], with ln_out
  const uint16_t* b;      // [C], with ln_out
  uint16_t* h_out;        // nullable
  uint16_t* ln_out;       // nullable
  int64_t rows, x_sn, y_sn, h_sn, ln_sn;
  float eps;
};

// fp32 -> 16-bit -> fp32 as a real rounding step.  Without the empty asm the
// compiler contracts `x + (float)(__bf16)(y * g)` into one FMA and skips the
// rounding between the product and the sum that the reference performs.
template <bool F16>
__device__ __forceinline__ float round16(float v) {
  uint32_t u = __builtin_bit_cast(uint16_t, f32_to_half<F16>(v));
  asm volatile("" : "+v"(u));
  return half_to_f32<F16>(__builtin_bit_cast(__bf16, (uint16_t)u));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

template <int NC, bool F16>  // C = 512 * NC
__global__ __launch_bounds__(64 * kRowsPerWG) void residual_layernorm_kernel(LnArgs a) {
  constexpr int C = 512 * NC;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWG + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // whole waves: no cross-wave exchange below

  float h[NC][8];
  const bf16x8* xr = reinterpret_cast<const bf16x8*>(a.x + row * a.x_sn) + lane;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const bf16x8 xv = xr[64 * i];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[i][e] = half_to_f32<F16>(xv[e]);
  }
  if (a.y != nullptr) {
    const bf16x8* yr = reinterpret_cast<const bf16x8*>(a.y + row * a.y_sn) + lane;
    const bf16x8* gr = reinterpret_cast<const bf16x8*>(a.gamma) + lane;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const bf16x8 yv = yr[64 * i], gv = gr[64 * i];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = round16<F16>(half_to_f32<F16>(yv[e]) * half_to_f32<F16>(gv[e]));
        h[i][e] = round16<F16>(h[i][e] + t);                   // 16-bit(x + 16-bit(gamma * y))
      }
    }
    if (a.h_out != nullptr) {
      bf16x8* hr = reinterpret_cast<bf16x8*>(a.h_out + row * a.h_sn) + lane;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        bf16x8 hv;
#pragma unroll
        for (int e = 0; e < 8; ++e) hv[e] = f32_to_half<F16>(h[i][e]);
        hr[64 * i] = hv;
      }
    }
  }
  if (a.ln_out == nullptr) return;

  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) s += h[i][e];
  const float mean = wave_sum(s) * (1.0f / C);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = h[i][e] - mean;
      ss = __builtin_fmaf(d, d, ss);
    }
  const float rstd = rsqrtf(wave_sum(ss) * (1.0f / C) + a.eps);
  const bf16x8* wr = reinterpret_cast<const bf16x8*>(a.w) + lane;
  const bf16x8* br = reinterpret_cast<const bf16x8*>(a.b) + lane;
  bf16x8* orow = reinterpret_cast<bf16x8*>(a.ln_out + row * a.ln_sn) + lane;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const bf16x8 wv = wr[64 * i], bv = br[64 * i];
    bf16x8 ov;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      ov[e] = f32_to_half<F16>(__builtin_fmaf((h[i][e] - mean) * rstd, half_to_f32<F16>(wv[e]),
                                              half_to_f32<F16>(bv[e])));
    orow[64 * i] = ov;
  }
}

}  // namespace
}  // namespace gpa

using namespace gpa;

namespace {

// Shared by the bf16 and fp16 entry points; `fn` names the entry point in
// error messages.
template <bool F16>
int ln_run(const char* fn, const void* x, const void* y, const void* gamma, const void* ln_weight,
           const void* ln_bias, float eps, int64_t rows, int64_t C, int64_t x_sn, int64_t y_sn,
           void* h_out, int64_t h_sn, void* ln_out, int64_t ln_sn, void* stream) {
  gpa_clear_error();
  if (rows < 0 || C < 0) {
    gpa_set_error("%s: negative size", fn);
    return GPA_E_INVALID;
  }
  if (C % 512 != 0 || C < 512 || C > 4096) {
    gpa_set_error("%s: C=%lld unsupported (multiple of 512, <= 4096)", fn, (long long)C);
    return GPA_E_UNSUPPORTED;
  }
  if (rows == 0) return GPA_OK;
  if (!x || (y && !gamma) || (ln_out && (!ln_weight || !ln_bias)) || (!h_out && !ln_out) ||
      (h_out && !y)) {
    gpa_set_error("%s: null pointer (x; gamma with y; weight and bias with ln_out; an output; "
                  "h_out only with y)", fn);
    return GPA_E_INVALID;
  }
  if (!(eps >= 0.f) || !isfinite(eps)) {
    gpa_set_error("%s: eps must be finite and >= 0", fn);
    return GPA_E_INVALID;
  }
  auto al16 = [](const void* p) { return (uintptr_t)p % 16 == 0; };
  const bool aligned = al16(x) && (!y || (al16(y) && al16(gamma))) &&
                       (!ln_out || (al16(ln_out) && al16(ln_weight) && al16(ln_bias))) &&
                       (!h_out || al16(h_out)) && (rows == 1 || x_sn % 8 == 0) &&
                       (!y || rows == 1 || y_sn % 8 == 0) && (!h_out || rows == 1 || h_sn % 8 == 0) &&
                       (!ln_out || rows == 1 || ln_sn % 8 == 0);
  if (!aligned) {
    gpa_set_error("%s: rows and parameters must be 16-byte aligned", fn);
    return GPA_E_INVALID;
  }
  const int64_t blocks = (rows + kRowsPerWG - 1) / kRowsPerWG;
  if (blocks > 0x7fffffff) {
    gpa_set_error("%s: too many rows", fn);
    return GPA_E_UNSUPPORTED;
  }
  LnArgs a{};
  a.x = (const uint16_t*)x;
  a.y = (const uint16_t*)y;
  a.gamma = (const uint16_t*)gamma;
  a.w = (const uint16_t*)ln_weight;
  a.b = (const uint16_t*)ln_bias;
  a.h_out = (uint16_t*)h_out;
  a.ln_out = (uint16_t*)ln_out;
  a.rows = rows;
  a.x_sn = x_sn; a.y_sn = y_sn; a.h_sn = h_sn; a.ln_sn = ln_sn;
  a.eps = eps;
  const dim3 grid((unsigned)blocks), block(64 * kRowsPerWG);
  const hipStream_t s = (hipStream_t)stream;
  switch (C / 512) {
#define GPA_LN_CASE(nc) \
  case nc: hipLaunchKernelGGL((residual_layernorm_kernel<nc, F16>), grid, block, 0, s, a); break;
    GPA_LN_CASE(1) GPA_LN_CASE(2) GPA_LN_CASE(3) GPA_LN_CASE(4)
    GPA_LN_CASE(5) GPA_LN_CASE(6) GPA_LN_CASE(7)
#undef GPA_LN_CASE
    default: hipLaunchKernelGGL((residual_layernorm_kernel<8, F16>), grid, block, 0, s, a); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("%s: launch failed: %s", fn, hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}

}  // namespace

#define GPA_LN_ARGS                                                                          \
  const void *x, const void *y, const void *gamma, const void *ln_weight, const void *ln_bias, \
      float eps, int64_t rows, int64_t C, int64_t x_sn, int64_t y_sn, void *h_out,           \
      int64_t h_sn, void *ln_out, int64_t ln_sn, void *stream
#define GPA_LN_PASS \
  x, y, gamma, ln_weight, ln_bias, eps, rows, C, x_sn, y_sn, h_out, h_sn, ln_out, ln_sn, stream

extern "C" int gpa_residual_layernorm_bf16(GPA_LN_ARGS) {
  return ln_run<false>("gpa_residual_layernorm_bf16", GPA_LN_PASS);
}

extern "C" int gpa_residual_layernorm_f16(GPA_LN_ARGS) {
  return ln_run<true>("gpa_residual_layernorm_f16", GPA_LN_PASS);
}
