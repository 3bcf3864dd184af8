// dtw_prep.hip — gfx950 kernels for the DTW alignment prep of WhisperDRZ.
//
// Replaces _dtw_prep_batch (src/whisperdrz/dtw_align.py:700-753) up to its device->host copy,
// including the median filter it calls (dtw_align.py:65-78 sort-based, 87-155 Triton):
//
//   in : W [B, H, T, A] fp32 raw cross-attention scores of the alignment heads
//        lens[B] valid text rows, caps[B] valid audio columns (int32, device)
//   out: M [B, T, C] fp32, C = min(max(caps), A)
//
//   p[b,h,t,:]  = softmax over columns c < caps[b] (others 0)            (dtw_align.py:724-727)
//   z[b,h,:,c]  = (p - mean_c) / sqrt(max(var_c, 1e-12)), where mean and var are taken over the
//                 rows t < lens[b] and divide by lens[b]; every row is normalised (729-738)
//   f[b,h,t,:]  = width-W median of z along c, reflect padding at 0 and A-1     (742-743)
//   M[b,t,c]    = mean over h of f, c < C                                      (745-746)
//
// Three launches, each HBM-bound on W (4 bytes per valid score), all reading only the valid
// columns c < caps[b]:
//   dtw_row_stats_kernel   one wave per row (b,h,t): online max / sum of exp2 -> (m, 1/l);
//                          16-byte loads when the rows are 16-byte aligned
//   dtw_col_stats_kernel   one workgroup per (b, h, 64 columns): the column's p values stay in
//                          registers (8 waves x up to 64 rows each) for an exact two-pass
//                          mean / variance -> (mean, 1/std)
//   dtw_filter_kernel      one workgroup per (b, 16 rows, 64 output columns): for each head the
//                          normalised tile with its +-PAD halo is built in LDS (the next head's
//                          scores are loaded while the current one is filtered), 4 medians per
//                          thread are accumulated in registers, and the head mean is stored once.
// A batch row whose cap or length is 0 yields NaN everywhere, as the reference's 0/0 does.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {
namespace {

constexpr int kColBlock = 64;   // columns per col-stats workgroup and per filter strip
constexpr int kFiltRows = 16;   // rows per filter workgroup
constexpr int kHalo = 8;        // LDS halo on each side of a filter strip (PAD <= 7)
constexpr int kTileCols = kColBlock + 2 * kHalo;  // 80
constexpr int kTilePitch = 84;  // floats; staggers rows across LDS banks
constexpr int kMaxRowsPerLane = kDtwMaxRows / 8;  // col stats: rows held per lane (8 waves)

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Softmax value of score x in a row with statistics (max*log2e, 1/sum). The column-statistics
// and filter kernels must compute bit-identical p for one score: a column whose valid rows are
// all equal has variance 0 and std 1e-6, so any difference would be amplified a million-fold.
// Contraction is off so the rounded product, not the exact one, meets the later subtraction.
__device__ __forceinline__ float softmax_value(float x, float2 st) {
#pragma clang fp contract(off)
  return exp2f(__builtin_fmaf(x, kLog2e, -st.x)) * st.y;
}

__device__ __forceinline__ int clamp_cap(int cap, int A) { return cap < 0 ? 0 : (cap > A ? A : cap); }

// ---------------------------------------------------------------------------------------------
// Row statistics: rs[(b*H + h)*T + t] = (max_c x*log2e, 1 / sum_c exp2(x*log2e - max)), c < cap.
// ---------------------------------------------------------------------------------------------
template <bool kVec>
__global__ __launch_bounds__(256) void dtw_row_stats_kernel(DtwArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t n_rows = (int64_t)a.B * a.H * a.T;
  if (row >= n_rows) return;
  const int t = (int)(row % a.T);
  const int bh = (int)(row / a.T);
  const int b = bh / a.H, h = bh % a.H;
  const int cap = clamp_cap(a.caps[b], a.A);
  const float* src = a.w + b * a.ws[0] + h * a.ws[1] + (int64_t)t * a.ws[2];

  float m = -INFINITY, s = 0.f;
  // kVec: rows start 16-byte aligned, 16-byte loads; otherwise 4-byte loads. Either way each
  // lane has 16 values in flight per iteration.
  constexpr int kPer = kVec ? 4 : 1;
  const int n_vec = cap / kPer;
  for (int j0 = lane; j0 < n_vec; j0 += 64 * 16 / kPer) {
    float x[16];
#pragma unroll
    for (int u = 0; u < 16 / kPer; ++u) {
      const int j = j0 + 64 * u;
      if constexpr (kVec) {
        f32x4 v = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        if (j < n_vec) v = reinterpret_cast<const f32x4*>(src)[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * u + i] = v[i];
      } else {
        x[u] = j < n_vec ? src[j] : -INFINITY;
      }
    }
    float mx = m;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      x[i] *= kLog2e;
      mx = fmaxf(mx, x[i]);
    }
    // mx is finite: the first element of this iteration is a valid column.
    s *= exp2f(m - mx);
    m = mx;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += exp2f(x[i] - m);
  }
  if constexpr (kVec) {
    // Tail columns [4*n_vec, cap), at most 3.
    const int c = 4 * n_vec + lane;
    if (lane < (cap & 3)) {
      const float x = src[c] * kLog2e;
      const float mx = fmaxf(m, x);
      s = s * exp2f(m - mx) + exp2f(x - mx);  // exp2(m - mx) is 0 when m = -inf and s = 0
      m = mx;
    }
  }
  const float M = wave_max(m);
  const float part = (s > 0.f) ? s * exp2f(m - M) : 0.f;
  const float l = wave_sum(part);
  if (lane == 0) {
    float2 r;
    r.x = M;
    r.y = 1.f / l;
    a.rs[row] = r;
  }
}

// ---------------------------------------------------------------------------------------------
// Column statistics over the valid rows: cs[(b*H + h)*A + c] = (mean, 1/sqrt(max(var, 1e-12))).
// Grid: (ceil(n_cols / 64), H, B) with n_cols = the columns the filter reads; (b, h) are
// visited last-to-first.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(512) void dtw_col_stats_kernel(DtwArgs a) {
  // Reverse order: the last scores the row pass streamed are still in the device-wide cache.
  const int b = a.B - 1 - (int)blockIdx.z, h = a.H - 1 - (int)blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cap = clamp_cap(a.caps[b], a.A);
  const int len = a.lens[b];
  const int c = blockIdx.x * kColBlock + lane;
  if (blockIdx.x * kColBlock >= cap || len <= 0) return;  // masked columns / NaN rows: not read
  const int rows = len < a.T ? len : a.T;
  const bool col_ok = c < cap;
  const int64_t bh = (int64_t)b * a.H + h;
  const float* src = a.w + b * a.ws[0] + h * a.ws[1] + c;
  const float2* rs = a.rs + bh * a.T;

  __shared__ float red[8][kColBlock];
  float p[kMaxRowsPerLane];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxRowsPerLane; ++i) {
    const int t = wave + 8 * i;
    p[i] = 0.f;
    if (t < rows && col_ok) {
      const float2 st = rs[t];
      p[i] = softmax_value(src[(int64_t)t * a.ws[2]], st);
      sum += p[i];
    }
  }
  red[wave][lane] = sum;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < 8; ++w) tot += red[w][lane];
  const float n = (float)len;
  const float mean = tot / n;
  __syncthreads();
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxRowsPerLane; ++i) {
    const int t = wave + 8 * i;
    if (t < rows) {
      const float d = p[i] - mean;
      sq += d * d;
    }
  }
  red[wave][lane] = sq;
  __syncthreads();
  if (wave == 0 && col_ok) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) v += red[w][lane];
    v = v / n;
    v = v < 1e-12f ? 1e-12f : v;
    float2 r;
    r.x = mean;
    r.y = 1.f / sqrtf(v);
    a.cs[bh * a.A + c] = r;
  }
}

// ---------------------------------------------------------------------------------------------
// Median selection. Any exact selection returns an element of the window, so the result equals
// the reference's sort / bubble-network median for finite inputs.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void cx(float& lo, float& hi) {
  const float a = fminf(lo, hi);
  hi = fmaxf(lo, hi);
  lo = a;
}

// Median of 7 with a 13-exchange selection network (verified on all 128 0-1 inputs).
__device__ __forceinline__ float median7(float p0, float p1, float p2, float p3, float p4, float p5,
                                         float p6) {
  cx(p0, p5); cx(p0, p3); cx(p1, p6); cx(p2, p4); cx(p0, p1); cx(p3, p5);
  cx(p2, p6); cx(p2, p3); cx(p3, p6); cx(p4, p5); cx(p1, p4);
  // The last two exchanges (1,3) and (3,4), of which only the middle output is used.
  return fminf(fmaxf(p1, p3), p4);
}

// Median of W (odd) by partial exchange sort: after W/2 + 1 passes that each carry the largest
// remaining element upwards, slot W/2 holds the median.
template <int W>
__device__ __forceinline__ float median_generic(float (&v)[W]) {
#pragma unroll
  for (int i = 0; i <= W / 2; ++i)
#pragma unroll
    for (int j = 0; j < W - 1 - i; ++j) cx(v[j], v[j + 1]);
  return v[W / 2];
}

template <int PAD>
__device__ __forceinline__ float window_median(const float* win) {  // win[0 .. 2*PAD]
  if constexpr (PAD == 0) {
    return win[0];
  } else if constexpr (PAD == 1) {
    return __builtin_amdgcn_fmed3f(win[0], win[1], win[2]);
  } else if constexpr (PAD == 3) {
    return median7(win[0], win[1], win[2], win[3], win[4], win[5], win[6]);
  } else {
    float v[2 * PAD + 1];
#pragma unroll
    for (int i = 0; i < 2 * PAD + 1; ++i) v[i] = win[i];
    return median_generic<2 * PAD + 1>(v);
  }
}

// ---------------------------------------------------------------------------------------------
// Normalise + median filter + head mean. Grid: (ceil(C / 64), ceil(T / 16), B), 256 threads.
// Load mapping: thread = (column j in [0, 80), row group g in [0, 3)); rows g, g+3, ... < 16.
// Filter mapping: thread = (row tid/16, output columns 4*(tid%16) .. +3).
// ---------------------------------------------------------------------------------------------
template <int PAD>
__global__ __launch_bounds__(256) void dtw_filter_kernel(DtwArgs a) {
  constexpr int kLoadRows = (kFiltRows + 2) / 3;  // 6
  const int b = blockIdx.z;
  const int t0 = blockIdx.y * kFiltRows;
  const int c0 = blockIdx.x * kColBlock;
  const int tid = threadIdx.x;
  const int cap = clamp_cap(a.caps[b], a.A);
  const int len = a.lens[b];

  const int fr = tid >> 4;       // filter row
  const int fq = 4 * (tid & 15);  // first of 4 output columns
  const int ot = t0 + fr;

  if (cap <= 0 || len <= 0) {  // 0/0 in the reference: the whole batch row is NaN
    if (ot < a.T)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c0 + fq + i < a.C) a.out[b * a.os[0] + (int64_t)ot * a.os[1] + c0 + fq + i] = __builtin_nanf("");
    return;
  }

  __shared__ float tile[kFiltRows * kTilePitch];
  __shared__ float2 rstat[kFiltRows];

  // Load-side column of this thread (tid < 240).
  const int lj = tid % kTileCols;
  const int lg = tid / kTileCols;  // 0..2 (3 for the 16 idle threads)
  int g = c0 - kHalo + lj;         // unreflected column
  // Only columns within +-PAD of an output column < C are read.
  const bool lneed = lg < 3 && lj >= kHalo - PAD && lj < kHalo + kColBlock + PAD && g < a.C + PAD;
  if (g < 0) g = -g;
  if (g >= a.A) g = 2 * (a.A - 1) - g;
  const bool lvalid = lneed && g < cap;  // g >= cap: p = 0, mean 0, z = 0

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float xv[kLoadRows];
  float2 cst = make_float2(0.f, 0.f);

  auto issue = [&](int h) {
    const float* src = a.w + b * a.ws[0] + h * a.ws[1] + g;
#pragma unroll
    for (int i = 0; i < kLoadRows; ++i) {
      const int r = lg + 3 * i;
      const int t = t0 + r;
      xv[i] = (lvalid && r < kFiltRows && t < a.T) ? src[(int64_t)t * a.ws[2]] : 0.f;
    }
    if (lvalid) cst = a.cs[((int64_t)b * a.H + h) * a.A + g];
  };

  issue(0);
  for (int h = 0; h < a.H; ++h) {
    // Row statistics of this head for the 16 rows.
    if (tid < kFiltRows) {
      const int t = t0 + tid;
      rstat[tid] = t < a.T ? a.rs[((int64_t)b * a.H + h) * a.T + t] : make_float2(0.f, 0.f);
    }
    __syncthreads();
    // Normalised tile: z = (exp2(x*log2e - m) / l - mean) / std.
    if (lg < 3) {
#pragma unroll
      for (int i = 0; i < kLoadRows; ++i) {
        const int r = lg + 3 * i;
        if (r < kFiltRows) {
          float z = 0.f;
          if (lvalid) {
            const float2 st = rstat[r];
            z = (softmax_value(xv[i], st) - cst.x) * cst.y;
          }
          tile[r * kTilePitch + lj] = z;
        }
      }
    }
    __syncthreads();
    if (h + 1 < a.H) issue(h + 1);  // next head's scores in flight during the filter
    // 4 medians from the LDS row segment [fq + kHalo - PAD, fq + 3 + kHalo + PAD].
    {
      float win[4 + 2 * PAD];
      const float* rowp = tile + fr * kTilePitch + fq + kHalo - PAD;
#pragma unroll
      for (int i = 0; i < 4 + 2 * PAD; ++i) win[i] = rowp[i];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += window_median<PAD>(win + i);
    }
    __syncthreads();  // the tile and rstat are rewritten for the next head
  }
  if (ot < a.T) {
    float* dst = a.out + b * a.os[0] + (int64_t)ot * a.os[1] + c0 + fq;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (c0 + fq + i < a.C) dst[i] = acc[i] / (float)a.H;
  }
}

}  // namespace

size_t dtw_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A) {
  const size_t rows = (size_t)(B * H * T) * sizeof(float2);
  const size_t cols = (size_t)(B * H * A) * sizeof(float2);
  return ((rows + 255) & ~(size_t)255) + cols;
}

void dtw_workspace_layout(void* ws, DtwArgs* a) {
  char* p = static_cast<char*>(ws);
  a->rs = reinterpret_cast<float2*>(p);
  const size_t rows = (size_t)((int64_t)a->B * a->H * a->T) * sizeof(float2);
  a->cs = reinterpret_cast<float2*>(p + ((rows + 255) & ~(size_t)255));
}

hipError_t launch_dtw_prep(const DtwArgs& a, hipStream_t stream) {
  const int64_t n_rows = (int64_t)a.B * a.H * a.T;
  if (n_rows == 0 || a.C == 0) return hipSuccess;
  const bool vec = (reinterpret_cast<uintptr_t>(a.w) & 15) == 0 && a.ws[0] % 4 == 0 && a.ws[1] % 4 == 0 &&
                   a.ws[2] % 4 == 0;
  const dim3 rgrid((unsigned)((n_rows + 3) / 4));
  if (vec) hipLaunchKernelGGL(dtw_row_stats_kernel<true>, rgrid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(dtw_row_stats_kernel<false>, rgrid, dim3(256), 0, stream, a);
  // Columns the filter reads: [0, min(A, C + pad)).
  const int need = a.C + a.pad < a.A ? a.C + a.pad : a.A;
  hipLaunchKernelGGL(dtw_col_stats_kernel, dim3((need + kColBlock - 1) / kColBlock, a.H, a.B), dim3(512), 0,
                     stream, a);
  const dim3 grid((a.C + kColBlock - 1) / kColBlock, (a.T + kFiltRows - 1) / kFiltRows, a.B);
  switch (a.pad) {
#define WDRZ_FILT(P) \
  case P:            \
    hipLaunchKernelGGL(dtw_filter_kernel<P>, grid, dim3(256), 0, stream, a); \
    break;
    WDRZ_FILT(0) WDRZ_FILT(1) WDRZ_FILT(2) WDRZ_FILT(3) WDRZ_FILT(4) WDRZ_FILT(5) WDRZ_FILT(6) WDRZ_FILT(7)
#undef WDRZ_FILT
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace wdrz
