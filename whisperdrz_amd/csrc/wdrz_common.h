// wdrz_common.h — device helpers shared by the gfx950 attention kernels.
//
// Element types are handled as raw 16-bit patterns (bf16 / fp16) or fp32; every load of a
// K/V/Q row slice is one 16-byte vector load, so a 64-wide head row is 128 B (8 lanes) in
// 16-bit types and 256 B (16 lanes) in fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wdrz {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 64;
constexpr float kLog2e = 1.4426950408889634f;
// Finite "minus infinity" for running maxima: exp2(x - kNegBig) never forms inf - inf.
constexpr float kNegBig = -1.0e30f;

struct Bf16 {};
struct F16 {};
struct F32 {};

template <typename T> struct ElemBytes;
template <> struct ElemBytes<Bf16> { static constexpr int value = 2; };
template <> struct ElemBytes<F16> { static constexpr int value = 2; };
template <> struct ElemBytes<F32> { static constexpr int value = 4; };

// ---- scalar conversions -------------------------------------------------------------------

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float f16_lo(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// Round-to-nearest-even fp32 -> bf16 for two values, packed lo | hi << 16.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t r;
  r.x = (__bf16)lo;
  r.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  f16x2_t r;
  r.x = (_Float16)lo;
  r.y = (_Float16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

// ---- 16-byte slices of a head row ---------------------------------------------------------
// A Slice holds the elements of one 16-byte load, widened to fp32.

template <typename T> struct Slice;

template <> struct Slice<Bf16> {
  static constexpr int N = 8;
  float v[8];
  __device__ __forceinline__ void from_raw(u32x4 r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_lo(r[i]);
      v[2 * i + 1] = bf16_hi(r[i]);
    }
  }
};
template <> struct Slice<F16> {
  static constexpr int N = 8;
  float v[8];
  __device__ __forceinline__ void from_raw(u32x4 r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = f16_lo(r[i]);
      v[2 * i + 1] = f16_hi(r[i]);
    }
  }
};
template <> struct Slice<F32> {
  static constexpr int N = 4;
  float v[4];
  __device__ __forceinline__ void from_raw(u32x4 r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(r[i]);
  }
};

// Store N fp32 values as one 16-byte slice of type T.
template <typename T> __device__ __forceinline__ u32x4 to_raw(const float* v);
template <> __device__ __forceinline__ u32x4 to_raw<Bf16>(const float* v) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
  return r;
}
template <> __device__ __forceinline__ u32x4 to_raw<F16>(const float* v) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_f16x2(v[2 * i], v[2 * i + 1]);
  return r;
}
template <> __device__ __forceinline__ u32x4 to_raw<F32>(const float* v) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = __float_as_uint(v[i]);
  return r;
}

__device__ __forceinline__ u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// Streaming load (nontemporal hint): for data read once per launch, such as the K/V rows a
// decode step walks. Measured on MI355X: +13% HBM throughput for the cross-attention stream.
__device__ __forceinline__ u32x4 load16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void store16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// ---- cross-lane reductions within groups of 8 / 16 consecutive lanes (DPP) ----------------
// quad_perm [1,0,3,2] = lane ^ 1, [2,3,0,1] = lane ^ 2, row_half_mirror pairs lane i with
// 7 - i inside each 8-lane half-row, row_mirror pairs lane i with 15 - i inside a 16-lane row.
// After the quad steps every lane of a quad holds the quad total, so a mirror step (which
// always pairs a lane with one in the other quad / other half) completes the group total.

__device__ __forceinline__ float dpp_xor1(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_xor2(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_half_mirror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               0x141, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_row_mirror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               0x140, 0xF, 0xF, false));
}

// Sum over each aligned group of G lanes (G = 8 or 16); every lane gets its group's total.
template <int G> __device__ __forceinline__ float group_sum(float x) {
  static_assert(G == 8 || G == 16, "group size");
  x += dpp_xor1(x);
  x += dpp_xor2(x);
  x += dpp_half_mirror(x);
  if constexpr (G == 16) x += dpp_row_mirror(x);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- XCD-aware work order ----------------------------------------------------------------------
// Work-group ids are dealt round-robin over the 8 XCDs. remap_xcd turns the id into a logical work
// index such that each XCD gets one contiguous range of logical indices: neighbouring work items
// (sharing inputs) then run on the same XCD and share its L2.
constexpr int kNumXcd = 8;
__device__ __forceinline__ int remap_xcd(int id, int n) {
  const int q = n / kNumXcd, rem = n % kNumXcd;
  const int xcd = id % kNumXcd, local = id / kNumXcd;
  return xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
}

}  // namespace wdrz
