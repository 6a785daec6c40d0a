// Internal interface between the attention entry points (attn_keybias.hip)
// and the kernel for head dims other than 64 (attn_any_dim.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gpa {

struct AnyDimArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const void* bias;       // GPA_BIAS_* kind chosen at launch; nullable for NONE
  uint16_t* o;
  float* lse;             // nullable
  int H;
  int64_t BH, M, N;
  int64_t q_sb, q_sh, q_sm, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn, o_sb, o_sh, o_sm;
  int64_t bias_sb, bias_sh, bias_sn;
  int64_t lse_sb, lse_sh;
  float c;                // sm_scale * log2(e)
  float mul;              // 1 / sm_scale
  float* ws;              // workspace (the bias rows of head dims 128 and 256)
  size_t ws_bytes;
};

// Head dims the kernels are built for: 16, 32, 128, 256.
bool attn_any_dim_supported(int64_t D);

// Workspace bytes a call at head dim D needs (the fp32 bias rows of the
// tiled kernel: B*H rows of N rounded up to 32 keys); at most the head-dim-64
// workspace of the same shape.
size_t attn_any_dim_ws_bytes(int64_t BH, int64_t N, int64_t D);

// Launch on `s`; returns hipGetLastError() of the launch.
template <bool F16>
hipError_t attn_any_dim_launch(const AnyDimArgs& a, int64_t D, int bias_kind, hipStream_t s);

}  // namespace gpa
