// Device helpers shared by the nvk kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nvk.h"

#define NVK_DEVICE __device__ __forceinline__

typedef __bf16 nvk_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 nvk_bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 nvk_bf16x2 __attribute__((ext_vector_type(2)));
typedef float nvk_f32x4 __attribute__((ext_vector_type(4)));
typedef float nvk_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t nvk_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t nvk_u32x2 __attribute__((ext_vector_type(2)));
typedef short nvk_i16x4 __attribute__((ext_vector_type(4)));
typedef short nvk_i16x8 __attribute__((ext_vector_type(8)));

// log2(e): softmax is evaluated as exp2(x*log2e - m), v_exp_f32 being base 2.
#define NVK_LOG2E 1.4426950408889634f

// ---- launch-status helper -------------------------------------------------
static inline int nvk_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NVK_OK : (int)e;
}

// ---- bf16 <-> f32 ----------------------------------------------------------
// bf16 is the high half of an f32: widening is a shift / mask.
NVK_DEVICE float nvk_bf16lo_to_f32(uint32_t w) { return __uint_as_float(w << 16); }
NVK_DEVICE float nvk_bf16hi_to_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even pack of two f32 into one bf16x2 word (v_cvt_pk_bf16_f32).
NVK_DEVICE uint32_t nvk_pack_bf16x2(float lo, float hi) {
  nvk_bf16x2 p = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, p);
}

// a.lo*b.lo + a.hi*b.hi + c with f32 accumulation (v_dot2_f32_bf16).
NVK_DEVICE float nvk_dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(nvk_bf16x2, a),
                                         __builtin_bit_cast(nvk_bf16x2, b), c, false);
}

// ---- 16-bit element types of q / K / V / outputs: bf16 or f16 --------------
// The attention kernels are written once over this trait: the packing of f32
// pairs (round to nearest even), the f32-accumulating pair dot product, the
// MFMA of the element type and the packed pair (1, 1) used for row sums.
typedef _Float16 nvk_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 nvk_f16x2 __attribute__((ext_vector_type(2)));

template <bool F16>
struct NvkElt;

template <>
struct NvkElt<false> {  // bf16
  typedef nvk_bf16x8 vec8;
  static constexpr uint32_t kOnes = 0x3F803F80u;
  static NVK_DEVICE uint32_t pack2(float lo, float hi) { return nvk_pack_bf16x2(lo, hi); }
  static NVK_DEVICE float dot2(uint32_t a, uint32_t b, float c) { return nvk_dot2_bf16(a, b, c); }
  static NVK_DEVICE uint16_t one(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
  // the low / high element of a packed pair, widened; x rounded to the type
  static NVK_DEVICE float lo(uint32_t w) { return nvk_bf16lo_to_f32(w); }
  static NVK_DEVICE float hi(uint32_t w) { return nvk_bf16hi_to_f32(w); }
  static NVK_DEVICE float round(float x) { return nvk_bf16hi_to_f32((uint32_t)one(x) << 16); }
  static NVK_DEVICE nvk_f32x16 mfma32x32x16(vec8 a, vec8 b, nvk_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static NVK_DEVICE nvk_f32x4 mfma16x16x32(vec8 a, vec8 b, nvk_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct NvkElt<true> {  // f16
  typedef nvk_f16x8 vec8;
  static constexpr uint32_t kOnes = 0x3C003C00u;
  static NVK_DEVICE uint32_t pack2(float lo, float hi) {
    nvk_f16x2 p = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, p);
  }
  static NVK_DEVICE float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(nvk_f16x2, a),
                                  __builtin_bit_cast(nvk_f16x2, b), c, false);
  }
  static NVK_DEVICE uint16_t one(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
  static NVK_DEVICE float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  static NVK_DEVICE float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  static NVK_DEVICE float round(float x) { return (float)(_Float16)x; }
  static NVK_DEVICE nvk_f32x16 mfma32x32x16(vec8 a, vec8 b, nvk_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static NVK_DEVICE nvk_f32x4 mfma16x16x32(vec8 a, vec8 b, nvk_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// ---- cross-lane reductions -------------------------------------------------
// DPP controls (GFX9 encoding): quad_perm xor1 / xor2, row_half_mirror, row_mirror.
#define NVK_DPP_QP_XOR1 0xB1
#define NVK_DPP_QP_XOR2 0x4E
#define NVK_DPP_HALF_MIRROR 0x141
#define NVK_DPP_MIRROR 0x140

template <int CTRL>
NVK_DEVICE float nvk_dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of LANES consecutive lanes (LANES in {4, 8, 16});
// every lane of the group receives the group total.
template <int LANES>
NVK_DEVICE float nvk_group_sum(float x) {
  static_assert(LANES == 4 || LANES == 8 || LANES == 16, "group size");
  x += nvk_dpp<NVK_DPP_QP_XOR1>(x);
  x += nvk_dpp<NVK_DPP_QP_XOR2>(x);
  if constexpr (LANES >= 8) x += nvk_dpp<NVK_DPP_HALF_MIRROR>(x);
  if constexpr (LANES >= 16) x += nvk_dpp<NVK_DPP_MIRROR>(x);
  return x;
}

// Value of lane (lane ^ MASK) for MASK in {16, 32} (ds_swizzle-free: bpermute).
template <int MASK>
NVK_DEVICE float nvk_xor_lane(float x) {
  const int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ MASK) << 2, __float_as_int(x)));
}

// max(a, b, c) as one v_max3_f32.  fmaxf would first quiet each operand
// (v_max x, x) since the MFMA results it reads are not known to be canonical;
// the scores here are never NaN unless the inputs are.
NVK_DEVICE float nvk_max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// max / sum of x over lanes l and l ^ 32, with v_permlane32_swap (a VALU
// exchange of the two wave halves, no LDS round trip).
NVK_DEVICE float nvk_max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
NVK_DEVICE float nvk_sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

NVK_DEVICE float nvk_fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- integer helpers ---------------------------------------------------------
// Page lookup for key position `pos` of a sequence: returns the flat cache row
// (page*block_size + offset) or -1 when the page id is outside [0, num_blocks).
NVK_DEVICE int64_t nvk_paged_row(const int32_t* __restrict__ bt_row, int pos, int block_size,
                                 int bs_shift, int num_blocks) {
  int logical, offset;
  if (bs_shift >= 0) {
    logical = pos >> bs_shift;
    offset = pos & (block_size - 1);
  } else {
    logical = pos / block_size;
    offset = pos - logical * block_size;
  }
  const int page = bt_row[logical];
  if (page < 0 || page >= num_blocks) return -1;
  return (int64_t)page * block_size + offset;
}

static inline int nvk_log2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((1 << s) < v) ++s;
  return s;
}

// ---- stream-K bookkeeping ----------------------------------------------------
// Last b in [0, B) with n * s_cs[b] <= c (s_cs non-decreasing, s_cs[0] = 0,
// c >= 0; B <= 4096), wave-uniform: the 64 lanes test every (B/64)-th entry,
// a ballot keeps the last that holds, and a second round tests the entries
// after it.  Two dependent LDS reads instead of a binary search's log2 B.
NVK_DEVICE int nvk_last_le(const int* s_cs, int B, int n, int64_t c, int lane) {
  const int stride = (B + 63) / 64;
  int b = lane * stride;
  bool p = b < B && (int64_t)n * s_cs[b] <= c;
  uint64_t m = __builtin_amdgcn_ballot_w64(p);  // lane 0 holds: s_cs[0] = 0
  int lo = (63 - __builtin_clzll(m)) * stride;
  if (stride > 1) {
    b = lo + lane;
    p = lane < stride && b < B && (int64_t)n * s_cs[b] <= c;
    m = __builtin_amdgcn_ballot_w64(p);  // lane 0 (b = lo) holds
    lo += 63 - __builtin_clzll(m);
  }
  return __builtin_amdgcn_readfirstlane(lo);
}

// Inclusive prefix sum over the 64 lanes of a wave in six DPP adds (row
// shifts by 1, 2, 4, 8 inside each 16-lane row, then the row totals carried
// by row_bcast:15 and row_bcast:31), no LDS round trip.  Equal to the
// __shfl_up scan for every input (integer adds).
NVK_DEVICE int nvk_wave_scan_add(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
  return x;
}
