// decode_ops.hip — the small per-step operations of the captured decode step, fused.
//
// 1. wdrz_add_layernorm: the residual add that closes a sub-layer and the LayerNorm that opens
//    the next one (src/whisperdrz/model.py:420-433: x = x + attn(attn_ln(x)); x = x +
//    cross_attn(cross_attn_ln(x)); x = x + mlp(mlp_ln(x)); the next block's attn_ln, or the
//    final ln, model.py:609-613). x += delta is rounded to the storage type as torch's add is;
//    the LayerNorm (eps 1e-5, affine) is computed in fp32 from the rounded sum, as torch's
//    LayerNorm does for 16-bit inputs, and rounded once. One wavefront per row; the row stays in
//    registers between the mean and the variance pass.
// 2. wdrz_masked_argmax: decode_batch's greedy sampling tail (src/whisperdrz/decoding.py:
//    1729-1761): masked = logits + (-65504 where blocked), then the repetition penalty
//    (x > 0 ? x / 1.2 : x * 1.2 where penalised), argmax. Each step rounds to the logits' type
//    as the torch ops do; ties go to the lowest index, as torch.argmax. One workgroup per row.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {
namespace {

template <typename T> struct Elem;
template <> struct Elem<Bf16> {
  static __device__ __forceinline__ float lo(uint32_t w) { return bf16_lo(w); }
  static __device__ __forceinline__ float hi(uint32_t w) { return bf16_hi(w); }
  static __device__ __forceinline__ uint32_t pack(float a, float b) { return pack_bf16x2(a, b); }
  static __device__ __forceinline__ float round(float v) { return (float)(__bf16)v; }
  static __device__ __forceinline__ float load1(const void* p, int64_t i) {
    return (float)static_cast<const __bf16*>(p)[i];
  }
};
template <> struct Elem<F16> {
  static __device__ __forceinline__ float lo(uint32_t w) { return f16_lo(w); }
  static __device__ __forceinline__ float hi(uint32_t w) { return f16_hi(w); }
  static __device__ __forceinline__ uint32_t pack(float a, float b) { return pack_f16x2(a, b); }
  static __device__ __forceinline__ float round(float v) { return (float)(_Float16)v; }
  static __device__ __forceinline__ float load1(const void* p, int64_t i) {
    return (float)static_cast<const _Float16*>(p)[i];
  }
};
template <> struct Elem<F32> {
  static __device__ __forceinline__ float round(float v) { return v; }
  static __device__ __forceinline__ float load1(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
  }
};

__device__ __forceinline__ float wave_sum64(float v) {
  v = group_sum<16>(v);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
}

// ---- residual add + LayerNorm (16-bit rows of n <= 64*8*NC elements) -------------------------
// NC = 16-byte chunks per lane (n <= 512 * NC). The LayerNorm weight and bias are loaded with the
// row, so the only dependent round trip is the row itself. NP > 0: the delta is a Linear's output
// given as NP fp32 split-K partials [NP][rows][n] plus its bias, rounded to the storage type
// after the sum, as the Linear's own output is.
template <typename T, int NC, int NP>
__global__ __launch_bounds__(256) void add_layernorm_kernel(AddLnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int nc = a.n >> 3;  // 8-element chunks
  char* xrow = static_cast<char*>(a.x) + row * a.x_stride * 2;
  const char* drow = NP ? nullptr : a.delta ? static_cast<const char*>(a.delta) + row * a.d_stride * 2 : nullptr;
  const bool has_delta = NP > 0 || drow != nullptr;
  u32x4 xw[NC], dw[NC], ww[NC], bw[NC];
  f32x4 pw[NC][NP > 0 ? 2 * NP : 1];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ci = lane + 64 * c;
    xw[c] = dw[c] = ww[c] = bw[c] = u32x4{0, 0, 0, 0};
    if (ci < nc) {
      xw[c] = *reinterpret_cast<const u32x4*>(xrow + ci * 16);
      if (drow) dw[c] = *reinterpret_cast<const u32x4*>(drow + ci * 16);
      if constexpr (NP > 0) {
        dw[c] = *reinterpret_cast<const u32x4*>(static_cast<const char*>(a.dbias) + ci * 16);
#pragma unroll
        for (int z = 0; z < NP; ++z) {
          const float* pr = a.dpart + ((int64_t)z * a.rows + row) * a.n + ci * 8;
          pw[c][2 * z] = *reinterpret_cast<const f32x4*>(pr);
          pw[c][2 * z + 1] = *reinterpret_cast<const f32x4*>(pr + 4);
        }
      }
      ww[c] = *reinterpret_cast<const u32x4*>(static_cast<const char*>(a.weight) + ci * 16);
      bw[c] = *reinterpret_cast<const u32x4*>(static_cast<const char*>(a.bias) + ci * 16);
    }
  }
  float v[NC][8];
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ci = lane + 64 * c;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[c][i] = 0.f;
    if (ci < nc) {
      float dl[8];
      if constexpr (NP > 0) {
        // the Linear's output: partials summed in split order, bias added, one rounding
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float t = pw[c][i >> 2][i & 3];
#pragma unroll
          for (int z = 1; z < NP; ++z) t += pw[c][2 * z + (i >> 2)][i & 3];
          const float bb = (i & 1) ? Elem<T>::hi(dw[c][i >> 1]) : Elem<T>::lo(dw[c][i >> 1]);
          dl[i] = Elem<T>::round(t + bb);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dl[2 * j] = Elem<T>::lo(dw[c][j]);
          dl[2 * j + 1] = Elem<T>::hi(dw[c][j]);
        }
      }
      u32x4 sw;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float s0 = Elem<T>::lo(xw[c][j]), s1 = Elem<T>::hi(xw[c][j]);
        if (has_delta) {
          s0 = Elem<T>::round(s0 + dl[2 * j]);
          s1 = Elem<T>::round(s1 + dl[2 * j + 1]);
          sw[j] = Elem<T>::pack(s0, s1);
        }
        v[c][2 * j] = s0;
        v[c][2 * j + 1] = s1;
        sum += s0 + s1;
      }
      if (has_delta) *reinterpret_cast<u32x4*>(xrow + ci * 16) = sw;  // the new residual
    }
  }
  const float inv_n = 1.f / (float)a.n;
  const float mean = wave_sum64(sum) * inv_n;
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (lane + 64 * c < nc)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = v[c][i] - mean;
        sq += d * d;
      }
  const float rstd = 1.f / sqrtf(wave_sum64(sq) * inv_n + a.eps);
  char* yrow = static_cast<char*>(a.y) + row * a.y_stride * 2;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ci = lane + 64 * c;
    if (ci < nc) {
      u32x4 yw;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float y0 = (v[c][2 * j] - mean) * rstd * Elem<T>::lo(ww[c][j]) + Elem<T>::lo(bw[c][j]);
        const float y1 = (v[c][2 * j + 1] - mean) * rstd * Elem<T>::hi(ww[c][j]) + Elem<T>::hi(bw[c][j]);
        yw[j] = Elem<T>::pack(y0, y1);
      }
      *reinterpret_cast<u32x4*>(yrow + ci * 16) = yw;
    }
  }
}

// ---- masked greedy sampling --------------------------------------------------------------
// argmax order of torch.argmax: NaN above every number (the first NaN wins), otherwise the
// larger value, ties to the lower index.
__device__ __forceinline__ bool argmax_beats(float v, int i, float b, int bi) {
  const bool vn = v != v, bn = b != b;
  if (vn != bn) return vn;
  if (vn) return i < bi;
  return v > b || (v == b && i < bi);
}

template <typename T>
__global__ __launch_bounds__(256) void masked_argmax_kernel(ArgmaxArgs a) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)row * a.l_stride;
  const uint8_t* bm = a.blocked ? a.blocked + (int64_t)row * a.m_stride : nullptr;
  const uint8_t* pm = a.penalty ? a.penalty + (int64_t)row * a.p_stride : nullptr;
  // -65504 in the logits' type, as the additive mask holds it (decoding.py:1736-1738)
  const float neg = Elem<T>::round(-65504.f);
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  for (int i = tid; i < a.V; i += 256) {
    float v = Elem<T>::load1(a.logits, base + i);
    v = Elem<T>::round(v + ((bm && bm[i]) ? neg : 0.f));  // logits + additive_mask
    if (pm && pm[i]) v = Elem<T>::round(v > 0.f ? v / 1.2f : v * 1.2f);
    if (argmax_beats(v, i, best, best_i)) {
      best = v;
      best_i = i;
    }
  }
  // workgroup argmax in the same order
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ob = __shfl_xor(best, o);
    const int oi = __shfl_xor(best_i, o);
    if (argmax_beats(ob, oi, best, best_i)) {
      best = ob;
      best_i = oi;
    }
  }
  __shared__ float sb[4];
  __shared__ int si[4];
  if ((tid & 63) == 0) {
    sb[tid >> 6] = best;
    si[tid >> 6] = best_i;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w)
      if (argmax_beats(sb[w], si[w], best, best_i)) {
        best = sb[w];
        best_i = si[w];
      }
    a.out[row] = best_i == 0x7fffffff ? 0 : best_i;
  }
}

}  // namespace

hipError_t launch_add_layernorm(int dtype, const AddLnArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  const dim3 grid((unsigned)((a.rows + 3) / 4));
  const int nc = (a.n + 511) / 512;
  const int np = a.dpart ? a.n_part : 0;
  // the partials form keeps 2 NP fp32 quads per chunk in registers: n <= 1536 (NC <= 3)
  if ((np != 0 && np != 2 && np != 4) || (np != 0 && nc > 3)) return hipErrorInvalidValue;
#define WDRZ_LN3(NC, NP)                                                                                 \
  if (dtype == 2) hipLaunchKernelGGL((add_layernorm_kernel<Bf16, NC, NP>), grid, dim3(256), 0, stream, a); \
  else hipLaunchKernelGGL((add_layernorm_kernel<F16, NC, NP>), grid, dim3(256), 0, stream, a);
#define WDRZ_LNP(NC)     \
  case NC:               \
    if (np == 0) {       \
      WDRZ_LN3(NC, 0)    \
    } else if (np == 2) { \
      WDRZ_LN3(NC, 2)    \
    } else {             \
      WDRZ_LN3(NC, 4)    \
    }                    \
    break;
#define WDRZ_LN(NC)   \
  case NC:            \
    WDRZ_LN3(NC, 0)   \
    break;
  switch (nc) {
    WDRZ_LNP(1) WDRZ_LNP(2) WDRZ_LNP(3) WDRZ_LN(4) WDRZ_LN(5) WDRZ_LN(6) WDRZ_LN(7) WDRZ_LN(8)
    default:
      return hipErrorInvalidValue;
  }
#undef WDRZ_LN
#undef WDRZ_LNP
#undef WDRZ_LN3
  return hipGetLastError();
}

hipError_t launch_masked_argmax(int dtype, const ArgmaxArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  const dim3 grid((unsigned)a.rows);
  if (dtype == 2) hipLaunchKernelGGL(masked_argmax_kernel<Bf16>, grid, dim3(256), 0, stream, a);
  else if (dtype == 1) hipLaunchKernelGGL(masked_argmax_kernel<F16>, grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(masked_argmax_kernel<F32>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace wdrz
