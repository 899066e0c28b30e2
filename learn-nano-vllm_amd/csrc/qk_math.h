// Per-head q/k RMSNorm + rotary embedding of one head row (head_dim 128),
// shared by the fused prologue kernel and the decode kernel that applies the
// prologue itself, so that both produce the same bits.
//
// Semantics (nanovllm/layers/layernorm.py:16-26, rotary_embedding.py:6-14),
// with T the model's element type (bf16 or f16, model_runner.py:29):
//   x = row.float(); x *= rsqrt(mean(x^2) + eps); x = T(x) * weight (T)
//   x1, x2 = halves of x; cos, sin = halves of cos_sin_cache[pos]
//   y1 = x1*cos - x2*sin ; y2 = x2*cos + x1*sin ; T(cat(y1, y2))
// Every f32 product and sum is rounded on its own (no fused multiply-add), as
// the reference's separate tensor operations do; a product of two T values
// is formed in f32 and rounded to T, as torch's elementwise kernels do.
//
// Lane mapping: a row group of 16 consecutive lanes owns the row, lane j
// holds elements 8j .. 8j+7 (16 bytes).  The sum of squares is a 16-lane DPP
// reduction; the rotation partner of element i (i +- 64) sits in lane j ^ 8
// of the same row group and comes through one DPP row rotation by 8.  All 16
// lanes of the row group must be active.
#pragma once

#include "nvk_common.h"

#define NVK_DPP_ROW_ROR8 0x128

namespace nvk_qk {

constexpr int kHD = 128;
constexpr int kLanesPerRow = kHD / 8;  // 16

// raw: this lane's 8 elements (T) of the head row; wraw: its 8 T of the norm
// weight; cs: the lane's cos[8(j%8) .. +7] (cs[0..1]) and sin[8(j%8) .. +7]
// (cs[2..3]) as f32.  Returns the lane's 8 rotated T, packed.  F16: T = f16,
// else bf16.
template <bool F16>
__device__ __forceinline__ nvk_u32x4 norm_rope8_cs(nvk_u32x4 raw, nvk_u32x4 wraw, float eps,
                                                   const nvk_u32x4 (&cs)[4], int j) {
#pragma clang fp contract(off)
  using E = NvkElt<F16>;
  float x[8];
  const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = E::lo(w4[i]);
    x[2 * i + 1] = E::hi(w4[i]);
  }
  // RMSNorm: var = mean(x^2) over the row (f32), x * rsqrt(var + eps) -> T,
  // then times the T weight -> T.
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  ss = nvk_group_sum<kLanesPerRow>(ss);
  const float rstd = rsqrtf(ss / (float)kHD + eps);
  const uint32_t ww[4] = {wraw.x, wraw.y, wraw.z, wraw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float n0 = E::round(x[2 * i] * rstd), n1 = E::round(x[2 * i + 1] * rstd);
    x[2 * i] = E::round(n0 * E::lo(ww[i]));
    x[2 * i + 1] = E::round(n1 * E::hi(ww[i]));
  }
  // Rotation: lanes 0-7 hold x1 (dims 0..63), lanes 8-15 x2 (dims 64..127).
  float cv[8], sv[8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t c4[4] = {cs[i].x, cs[i].y, cs[i].z, cs[i].w};
    const uint32_t s4[4] = {cs[2 + i].x, cs[2 + i].y, cs[2 + i].z, cs[2 + i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cv[4 * i + e] = __uint_as_float(c4[e]);
      sv[4 * i + e] = __uint_as_float(s4[e]);
    }
  }
  const bool first_half = j < kLanesPerRow / 2;
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float other = nvk_dpp<NVK_DPP_ROW_ROR8>(x[e]);
    const float a0 = x[e] * cv[e];
    const float a1 = other * sv[e];
    y[e] = first_half ? a0 - a1 : a0 + a1;  // x1*cos - x2*sin | x2*cos + x1*sin
  }
  nvk_u32x4 out;
  out.x = E::pack2(y[0], y[1]);
  out.y = E::pack2(y[2], y[3]);
  out.z = E::pack2(y[4], y[5]);
  out.w = E::pack2(y[6], y[7]);
  return out;
}

// The same with the cos/sin row read here: cs is the position's row (64 cos
// then 64 sin, f32).
template <bool F16>
__device__ __forceinline__ nvk_u32x4 norm_rope8(nvk_u32x4 raw, nvk_u32x4 wraw, float eps,
                                                const float* cs, int j) {
  const float* c = cs + 8 * (j & 7);
  const nvk_u32x4 v[4] = {*reinterpret_cast<const nvk_u32x4*>(c),
                          *reinterpret_cast<const nvk_u32x4*>(c + 4),
                          *reinterpret_cast<const nvk_u32x4*>(c + kHD / 2),
                          *reinterpret_cast<const nvk_u32x4*>(c + kHD / 2 + 4)};
  return norm_rope8_cs<F16>(raw, wraw, eps, v, j);
}

}  // namespace nvk_qk
