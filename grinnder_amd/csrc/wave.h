// Cross-lane sums and maxima of a 64-lane gfx950 wavefront without the LDS
// crossbar: DPP within rows of 16 lanes (quad_perm, row_half_mirror,
// row_mirror, row_ror:8) and the gfx950 v_permlane16_swap /
// v_permlane32_swap across rows.  Each step combines a lane with its partner
// by a commutative operation, so every lane of a group ends with the same
// bits, and the order is fixed, so results do not vary between runs.
//
// Call these with all 64 lanes active (uniform control flow).
#pragma once

#include <hip/hip_runtime.h>

namespace gr_wave {

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Value of lane ^ 16 (rows 0 <-> 1, 2 <-> 3), through v_permlane16_swap.
__device__ __forceinline__ float xor16(float v) {
  const int x = __builtin_bit_cast(int, v);
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  // r[0] holds rows (0, 0, 2, 2) and r[1] rows (1, 1, 3, 3) of x.
  return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}

// Value of lane ^ 32, through v_permlane32_swap.
__device__ __forceinline__ float xor32(float v) {
  const int x = __builtin_bit_cast(int, v);
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  // r[0] holds halves (0, 0) and r[1] halves (1, 1) of x.
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}

// Sum over aligned groups of G consecutive lanes (G a power of two, 1..64);
// every lane of a group gets the group's sum.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "G must be a power of two <= 64");
  if constexpr (G >= 2) v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (G >= 4) v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (G >= 8) v += dpp<0x141>(v);  // row_half_mirror: the other quad
  if constexpr (G >= 16) v += dpp<0x140>(v); // row_mirror: the other half-row
  if constexpr (G >= 32) v += xor16(v);
  if constexpr (G >= 64) v += xor32(v);
  return v;
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
  static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "G must be a power of two <= 64");
  if constexpr (G >= 2) v = fmaxf(v, dpp<0xB1>(v));
  if constexpr (G >= 4) v = fmaxf(v, dpp<0x4E>(v));
  if constexpr (G >= 8) v = fmaxf(v, dpp<0x141>(v));
  if constexpr (G >= 16) v = fmaxf(v, dpp<0x140>(v));
  if constexpr (G >= 32) v = fmaxf(v, xor16(v));
  if constexpr (G >= 64) v = fmaxf(v, xor32(v));
  return v;
}

__device__ __forceinline__ int xor16_int(int x) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  return (threadIdx.x & 16) ? r[0] : r[1];
}

__device__ __forceinline__ int xor32_int(int x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return (threadIdx.x & 32) ? r[0] : r[1];
}

template <int CTRL>
__device__ __forceinline__ int dpp_int(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}

// Minimum over aligned groups of G consecutive lanes, for ints.
template <int G>
__device__ __forceinline__ int group_min_int(int v) {
  static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "G must be a power of two <= 64");
  if constexpr (G >= 2) v = min(v, dpp_int<0xB1>(v));
  if constexpr (G >= 4) v = min(v, dpp_int<0x4E>(v));
  if constexpr (G >= 8) v = min(v, dpp_int<0x141>(v));
  if constexpr (G >= 16) v = min(v, dpp_int<0x140>(v));
  if constexpr (G >= 32) v = min(v, xor16_int(v));
  if constexpr (G >= 64) v = min(v, xor32_int(v));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }

// Sum over the lanes that share lane % G (the 64 / G edge slots of G lanes
// each, G in 8..64); every such lane gets the sum.
template <int G>
__device__ __forceinline__ float slot_sum(float v) {
  static_assert(G >= 8 && G <= 64 && (G & (G - 1)) == 0, "G must be 8, 16, 32 or 64");
  if constexpr (G <= 8) v += dpp<0x128>(v);  // row_ror:8 = lane ^ 8 within a row
  if constexpr (G <= 16) v += xor16(v);
  if constexpr (G <= 32) v += xor32(v);
  return v;
}

// 4 x 4 transpose across the wavefront's four 16-lane rows: afterwards
// component j of lane l of row r holds what component r of lane l of row j
// held.  One round of v_permlane32_swap (rows 0-1 against 2-3) on the
// component pairs (x, z), (y, w), one of v_permlane16_swap (rows 0, 2
// against 1, 3) on (x, y), (z, w).
// (The result's elements are copied to ints before the bit casts: a bit cast
// of a vector element read element 0's storage for both with this compiler.)
__device__ __forceinline__ void swap_rows32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, a),
                                                  __builtin_bit_cast(int, b), false, false);
  const int r0 = r[0], r1 = r[1];
  a = __builtin_bit_cast(float, r0);  // rows (a0, a1, b0, b1)
  b = __builtin_bit_cast(float, r1);  // rows (a2, a3, b2, b3)
}

__device__ __forceinline__ void swap_rows16(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, a),
                                                  __builtin_bit_cast(int, b), false, false);
  const int r0 = r[0], r1 = r[1];
  a = __builtin_bit_cast(float, r0);  // rows (a0, b0, a2, b2)
  b = __builtin_bit_cast(float, r1);  // rows (a1, b1, a3, b3)
}

__device__ __forceinline__ void row_transpose4(float4& v) {
  swap_rows32(v.x, v.z);
  swap_rows32(v.y, v.w);
  swap_rows16(v.x, v.y);
  swap_rows16(v.z, v.w);
}

// 4 x 4 transpose across each lane quad (c = lane & 3): lane c ends with
// element j = lane j's element c.  Each round swaps, with the partner lane
// (lane ^ 1, then lane ^ 2), the elements whose index bit differs from the
// lane's.  A v_mfma_f32_16x16x4_f32 result (lane holds rows 4 (lane / 16) + q
// of column lane % 16) becomes four consecutive columns of one row per lane.
__device__ __forceinline__ void quad_transpose(float& v0, float& v1, float& v2, float& v3,
                                               int c) {
  {
    const bool hi = c & 1;
    const float r0 = dpp<0xB1>(hi ? v0 : v1);  // quad_perm [1,0,3,2]
    const float r2 = dpp<0xB1>(hi ? v2 : v3);
    if (hi) {
      v0 = r0;
      v2 = r2;
    } else {
      v1 = r0;
      v3 = r2;
    }
  }
  {
    const bool hi = c & 2;
    const float r0 = dpp<0x4E>(hi ? v0 : v2);  // quad_perm [2,3,0,1]
    const float r1 = dpp<0x4E>(hi ? v1 : v3);
    if (hi) {
      v0 = r0;
      v1 = r1;
    } else {
      v2 = r0;
      v3 = r1;
    }
  }
}

// Raw buffer stores.  A store whose byte offset is at or past the resource's
// size is dropped by the hardware, so a kernel can send the rows or lanes it
// must not write past the end instead of branching around the store; with no
// branch the compiler knows how many stores are in flight and can wait for a
// later load without waiting for them.  Word 3 of the resource is the gfx9
// family's raw-buffer format (the value composable_kernel's ck.hpp uses).
constexpr uint32_t kBufferDrop = 0x80000000u;  // past any resource made below

// `bytes` < 2^31; the base must be wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ void buffer_store(__amdgpu_buffer_rsrc_t r, uint32_t offset,
                                             float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, offset, 0, 0);
}

}  // namespace gr_wave
