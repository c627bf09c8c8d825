// Shared device helpers for the gfx950 INT8 decode-attention library.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include <string>

#include "../../include/flashspec_hip.h"

namespace fs {

constexpr int kWave = 64;       // CDNA wavefront width
constexpr int kTile = 16;       // tokens per decode tile (one 16-token quant block)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -3.0e38f;  // finite stand-in for -inf in running maxima

// ---- host-side error state (defined in fs_capi.hip) --------------------------------------
int set_error(int code, const std::string& msg);
int check_launch(const char* what);

// ---- dtype helpers ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__half x) { return __half2float(x); }
__device__ __forceinline__ float to_f32(__hip_bfloat16 x) { return __bfloat162float(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ __half from_f32<__half>(float x) { return __float2half_rn(x); }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float x) {
  return __float2bfloat16(x);
}

// ---- cross-lane helpers -------------------------------------------------------------------------
// DPP row controls (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes (N in 1,2,4,8,16); every lane of a group gets the
// same bits because each step adds two commutative operands.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
  if constexpr (N >= 2) x += dpp_f32<kDppQuadXor1>(x);
  if constexpr (N >= 4) x += dpp_f32<kDppQuadXor2>(x);
  if constexpr (N >= 8) x += dpp_f32<kDppRowHalfMirror>(x);
  if constexpr (N >= 16) x += dpp_f32<kDppRowMirror>(x);
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, kWave));
  return x;
}
__device__ __forceinline__ float wave_min(float x) {
  for (int off = 32; off > 0; off >>= 1) x = fminf(x, __shfl_xor(x, off, kWave));
  return x;
}

// ---- gfx950 lane swaps (VALU; no LDS traffic) ----------------------------------------------------
// For registers x and y of every lane (layouts checked lane by lane on gfx950):
//   swap32: .a = x of lanes 0-31 in lanes 0-31, y of lanes 0-31 in lanes 32-63;
//           .b = x of lanes 32-63 in lanes 0-31, y of lanes 32-63 in lanes 32-63.
//   swap16 (rows of 16 lanes r0..r3): .a = (x.r0, y.r0, x.r2, y.r2); .b = (x.r1, y.r1, x.r3, y.r3).
// So swap(x, y).a + swap(x, y).b is the sum over the partner rows of x in the lower rows and of y
// in the upper ones (one half of a reduce-scatter), and swap(x, x) gives every lane the same sum.
struct LanePair {
  float a, b;
};
__device__ __forceinline__ LanePair swap32(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, y),
                                                  false, false);
  return {__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1])};
}
__device__ __forceinline__ LanePair swap16(float x, float y) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, y),
                                                  false, false);
  return {__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1])};
}
constexpr int kDppRowRor8 = 0x128;  // lane i of a row reads lane (i + 8) % 16
// lane i reads lane i ^ 4 (ds_swizzle bit-mask mode: and 0x1f, or 0, xor 4; no memory access)
__device__ __forceinline__ float swizzle_xor4(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x101f));
}

// Maximum over the whole wave, every lane getting the same bits.
__device__ __forceinline__ float wave_max_valu(float x) {
  x = fmaxf(x, dpp_f32<kDppQuadXor1>(x));
  x = fmaxf(x, dpp_f32<kDppQuadXor2>(x));
  x = fmaxf(x, dpp_f32<kDppRowHalfMirror>(x));
  x = fmaxf(x, dpp_f32<kDppRowMirror>(x));
  const LanePair r16 = swap16(x, x);
  x = fmaxf(r16.a, r16.b);
  const LanePair r32 = swap32(x, x);
  return fmaxf(r32.a, r32.b);
}

// Minimum over the whole wave, every lane getting the same bits.
__device__ __forceinline__ float wave_min_valu(float x) {
  x = fminf(x, dpp_f32<kDppQuadXor1>(x));
  x = fminf(x, dpp_f32<kDppQuadXor2>(x));
  x = fminf(x, dpp_f32<kDppRowHalfMirror>(x));
  x = fminf(x, dpp_f32<kDppRowMirror>(x));
  const LanePair r16 = swap16(x, x);
  x = fminf(r16.a, r16.b);
  const LanePair r32 = swap32(x, x);
  return fminf(r32.a, r32.b);
}

// Sum over the whole wave, every lane getting the same bits: each step adds the same two
// operands in both lanes of a partner pair (and addition commutes).
__device__ __forceinline__ float wave_sum_valu(float x) {
  x = group_sum<16>(x);
  const LanePair r16 = swap16(x, x);
  x = r16.a + r16.b;
  const LanePair r32 = swap32(x, x);
  return r32.a + r32.b;
}

__device__ __forceinline__ int readlane_i32(int x, int lane) { return __builtin_amdgcn_readlane(x, lane); }
__device__ __forceinline__ float readlane_f32(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// x / scale correctly rounded, from rcp = RN(1 / scale) and one FMA correction step
// (Markstein's theorem: with rcp correctly rounded and q0 = RN(x * rcp) within one ulp,
// r = x - q0 * scale is exact and RN(q0 + r * rcp) = RN(x / scale)).  A brute-force check
// over every fp16 input and random fp32 inputs against IEEE division (tests/cdiv) finds no
// difference except the sign of a zero quotient, which `+ zero` erases.  Valid while
// x * rcp stays finite; the caller checks that once per group.
__device__ __forceinline__ float div_by_scale(float x, float scale, float rcp) {
  const float q0 = x * rcp;
  const float r = __builtin_fmaf(-q0, scale, x);
  return __builtin_fmaf(r, rcp, q0);
}

}  // namespace fs
