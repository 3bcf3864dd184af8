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
// One workgroup per (256 audio columns, 32 text rows, b*H + h), 4 wavefronts, each a 32 x 64
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

constexpr int kQkRows = 32;   // text rows per workgroup (one MFMA row tile)
constexpr int kQkCols = 256;  // audio columns per workgroup (64 per wavefront)
constexpr int kQkPitch = kQkCols + 4;

// v_mfma_f32_32x32x16 operand layouts (lane l): A row l%32, k 8*(l/32) .. +8; B column l%32,
// k 8*(l/32) .. +8; C element i: row 8*(i/4) + 4*(l/32) + i%4, column l%32.
// The 32 x 256 fp32 block is staged in LDS and written as whole 1 KB row segments (one 16-byte
// store per lane), streamed past the caches: the kernel's cost is this write.
template <typename T>
__global__ __launch_bounds__(256) void dtw_qk_kernel(DtwQkArgs a) {
  typedef typename Mfma32<T>::op_t op_t;
  __shared__ float stage[kQkRows * kQkPitch];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Logical order: column blocks fastest (the workgroups writing one 32-row band of the output,
  // 6 KB rows at A = 1500, run back to back: 107 -> 100 us against row blocks fastest), then row
  // blocks, then (b, h); remapped so that each XCD takes a contiguous range, and a (b, h)'s K
  // blocks stay in that XCD's L2.
  const int n_rb = (a.T + kQkRows - 1) / kQkRows, n_cb = (a.A + kQkCols - 1) / kQkCols;
  const int tile = remap_xcd(blockIdx.x, gridDim.x);
  const int cb = tile % n_cb, rb = (tile / n_cb) % n_rb, bh = tile / (n_rb * n_cb);
  const int b = bh / a.H, h = bh % a.H;
  const int r0 = rb * kQkRows;
  const int c0 = cb * kQkCols;
  const int kh = 8 * (lane >> 5);  // this lane's 8 of every 16 head dimensions

  // Rows / columns past the end are clamped to the last one (valid addresses); their results
  // are not stored.
  const int t = min(r0 + (lane & 31), a.T - 1);
  const char* qrow = static_cast<const char*>(a.q[h]) + (b * a.qs[0] + (int64_t)t * a.qs[1]) * 2;
  op_t qa[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qa[ks] = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(qrow + (16 * ks + kh) * 2));

#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int cl = 64 * wave + 32 * j + (lane & 31);  // column within the block
    const int col = min(c0 + cl, a.A - 1);
    const char* krow = static_cast<const char*>(a.k[h]) + (b * a.ks[0] + (int64_t)col * a.ks[1]) * 2;
    op_t kb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      kb[ks] = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(krow + (16 * ks + kh) * 2));
    f32x16 acc = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = Mfma32<T>::run(qa[ks], kb[ks], acc);
#pragma unroll
    for (int i = 0; i < 16; ++i) stage[(8 * (i / 4) + 4 * (lane >> 5) + (i % 4)) * kQkPitch + cl] = acc[i] * a.scale2;
  }
  __syncthreads();

  float* out = a.out + b * a.os[0] + h * a.os[1];
  const int cl = 4 * lane;  // this lane's 4 columns of a row segment
  const int col = c0 + cl;
#pragma unroll
  for (int rr = 0; rr < kQkRows / 4; ++rr) {
    const int row = 4 * rr + wave;
    if (r0 + row < a.T) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(stage + row * kQkPitch + cl);
      float* dst = out + (int64_t)(r0 + row) * a.os[2] + col;
      if (a.vec && col + 4 <= a.A) {
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(dst));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (col + i < a.A) dst[i] = v[i];
      }
    }
  }
}

}  // namespace

hipError_t launch_dtw_qk(int dtype, DtwQkArgs a, hipStream_t stream) {
  if (a.B == 0 || a.T == 0 || a.A == 0) return hipSuccess;
  a.vec = (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 && a.os[0] % 4 == 0 && a.os[1] % 4 == 0 &&
          a.os[2] % 4 == 0;
  const int64_t n = (int64_t)((a.A + kQkCols - 1) / kQkCols) * ((a.T + kQkRows - 1) / kQkRows) * a.B * a.H;
  if (n > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)n);
  if (dtype == 2) hipLaunchKernelGGL(dtw_qk_kernel<Bf16>, grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(dtw_qk_kernel<F16>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace wdrz
