// dtw_qk.hip — gfx950 kernel for the alignment heads' raw cross-attention scores.
//
// Replaces CrossAttnCapture.compute_attention (src/whisperdrz/dtw_align.py:553-586):
//   S[b, h, t, a] = sum_d (Q_h[b, t, d] * s) * (K_h[b, a, d] * s),  s = head_dim^-0.25,
// where Q_h / K_h are head slices of the captured query / key projections of the decoder layers
// that hold the selected heads (no softmax). The reference gathers the slices with
// torch.stack(...).float() and runs one fp32 batched matmul; here each head slice is read in
// place (per-head base pointers, shared strides) in bf16 / fp16 and multiplied on the matrix
// cores with fp32 accumulation (products of 16-bit values are exact in fp32), then scaled by s^2.
//
// One workgroup per (128 audio columns, 64 text rows, b*H + h), 4 wavefronts, each a 32 x 64
// output block as two 32x32 tiles of v_mfma_f32_32x32x16 over the 64-dim head (4 k-steps).
// Operands come straight from global memory as 16-byte row slices (a Q row and a K row are
// 128 contiguous bytes); the result is written as fp32, which is what bounds the kernel (HBM).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {
namespace {

template <typename T> struct Mfma32;
template <> struct Mfma32<Bf16> {
  typedef bf16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma32<F16> {
  typedef f16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kQkRows = 64;   // text rows per workgroup
constexpr int kQkCols = 128;  // audio columns per workgroup

// v_mfma_f32_32x32x16 operand layouts (lane l): A row l%32, k 8*(l/32) .. +8; B column l%32,
// k 8*(l/32) .. +8; C element i: row 8*(i/4) + 4*(l/32) + i%4, column l%32.
template <typename T>
__global__ __launch_bounds__(256) void dtw_qk_kernel(DtwQkArgs a) {
  typedef typename Mfma32<T>::op_t op_t;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int bh = blockIdx.z;
  const int b = bh / a.H, h = bh % a.H;
  const int r0 = blockIdx.y * kQkRows + 32 * (wave & 1);
  const int c0 = blockIdx.x * kQkCols + 64 * (wave >> 1);
  const int kh = 8 * (lane >> 5);  // this lane's 8 of every 16 head dimensions

  // Rows / columns past the end are clamped to the last one (valid addresses); their results
  // are not stored.
  const int t = min(r0 + (lane & 31), a.T - 1);
  const char* qrow = static_cast<const char*>(a.q[h]) + (b * a.qs[0] + (int64_t)t * a.qs[1]) * 2;
  op_t qa[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qa[ks] = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(qrow + (16 * ks + kh) * 2));

  f32x16 acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = min(c0 + 32 * j + (lane & 31), a.A - 1);
    const char* krow = static_cast<const char*>(a.k[h]) + (b * a.ks[0] + (int64_t)col * a.ks[1]) * 2;
    op_t kb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      kb[ks] = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(krow + (16 * ks + kh) * 2));
    acc[j] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc[j] = Mfma32<T>::run(qa[ks], kb[ks], acc[j]);
  }

  float* out = a.out + b * a.os[0] + h * a.os[1];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = c0 + 32 * j + (lane & 31);
    if (col < a.A) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = r0 + 8 * (i / 4) + 4 * (lane >> 5) + (i % 4);
        if (row < a.T) out[(int64_t)row * a.os[2] + col] = acc[j][i] * a.scale2;
      }
    }
  }
}

}  // namespace

hipError_t launch_dtw_qk(int dtype, const DtwQkArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.T == 0 || a.A == 0) return hipSuccess;
  const dim3 grid((a.A + kQkCols - 1) / kQkCols, (a.T + kQkRows - 1) / kQkRows, a.B * a.H);
  if (dtype == 2) hipLaunchKernelGGL(dtw_qk_kernel<Bf16>, grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(dtw_qk_kernel<F16>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace wdrz
