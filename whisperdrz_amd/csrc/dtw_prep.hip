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
// Width 7 (the reference's) with A >= 256, the path of every Whisper window: the statistics
// in one pass (dtw_rowcol_kernel + dtw_col_merge_kernel, rows 16-byte aligned, A <= 2048)
// and the filter in dtw_seg_kernel (one wavefront per 4 rows x 250 columns, no workgroup
// barriers). Other widths and shapes take dtw_band_kernel (rows 16-byte aligned,
// A <= 2048) or the three column-strip launches below.
// The column-strip launches, each HBM-bound on W (4 bytes per valid score), all reading only
// the valid columns c < caps[b]:
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

#include <type_traits>

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

// Wave-wide reductions without LDS round trips: DPP inside each 16-lane row (lane ^ 1, ^ 2, then
// the half-row and row mirrors), then the gfx950 row swaps across the four rows.
__device__ __forceinline__ float swap_max(float x) {
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_xor1(v));
  v = fmaxf(v, dpp_xor2(v));
  v = fmaxf(v, dpp_half_mirror(v));
  v = fmaxf(v, dpp_row_mirror(v));
  return swap_max(v);
}
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
}

// Softmax value of score x in a row with statistics (max*log2e, 1/sum). The column-statistics
// and filter kernels must compute bit-identical p for one score: a column whose valid rows are
// all equal has variance 0 and std 1e-6, so any difference would be amplified a million-fold.
// Contraction is off so the rounded product, not the exact one, meets the later subtraction.
__device__ __forceinline__ float softmax_scale_e(float e, float rl) {
#pragma clang fp contract(off)
  return e * rl;
}
// The hardware exp2 (no denormal-range fix-up: a value below 2^-126 is negligible next to the
// column mean it is compared with).
__device__ __forceinline__ float softmax_exp(float x, float m) { return fast_exp2(__builtin_fmaf(x, kLog2e, -m)); }
__device__ __forceinline__ float softmax_value(float x, float2 st) {
  return softmax_scale_e(softmax_exp(x, st.x), st.y);
}
// The same for an unscaled score x whose softmax argument is x * c (c = scale^2 * log2e for the
// fused path's raw Q.K products): the scale rides in the FMA instead of a multiply per score.
__device__ __forceinline__ float softmax_exp_c(float x, float c, float m) { return fast_exp2(__builtin_fmaf(x, c, -m)); }
__device__ __forceinline__ float softmax_value_c(float x, float c, float2 st) {
  return softmax_scale_e(softmax_exp_c(x, c, st.x), st.y);
}

// f(0), f(1), ..., f(N-1) as straight-line code.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(N - 1);
  }
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
    a.cs[bh * a.cpitch + c] = r;
  }
}

// ---------------------------------------------------------------------------------------------
// Fused row + column statistics (rows 16-byte aligned, A <= 256*NK): one workgroup per
// (64-row chunk, h, b), 4 waves x 16 rows. A wave holds a whole row in registers (NK 16-byte
// loads per lane, the next row's loads in flight), reduces its max and sum across the wave,
// stores the row statistics, and folds the row's softmax values into per-column Welford
// accumulators (mean, M2) when the row is valid. The 4 waves' accumulators are merged (Chan)
// through LDS and the chunk's partial (mean, M2) per column is stored for dtw_col_merge_kernel.
// ---------------------------------------------------------------------------------------------
constexpr int kRcWaves = 4;
// Workgroups that fit on the GPU at once: 256 CUs x 3 four-wave workgroups at up to 168 VGPRs
// (the workspace's chunking and the fused pass's), x 2 at up to 256 (dtw_rowcol_kernel). The
// rows of each (b, h) are cut into as many chunks as keep B*H*chunks within one such round, so
// no workgroup runs in a second, mostly idle round.
constexpr int kRcSlots = 768;
constexpr int kRcSlotsRowcol = 512;
// Bytes of W the statistics pass leaves in the Infinity Cache for the filter pass.
constexpr int64_t kMallKeepBytes = 224ll << 20;

__device__ __forceinline__ void chan_merge(float na, float& ma, float& qa, float nb, float mb, float qb) {
  if (nb == 0.f) return;
  const float n = na + nb;
  const float d = mb - ma;
  ma += d * (nb / n);
  qa += qb + d * d * (na * nb / n);
}

template <int NK, bool NT>
__device__ __attribute__((always_inline)) inline void rowcol_body(const DtwArgs& a, int chunk, int h, int b) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cap = clamp_cap(a.caps[b], a.A);
  const int len = a.lens[b];
  if (cap <= 0 || len <= 0) return;  // the filter writes NaN for this batch row
  const int rows_valid = len < a.T ? len : a.T;
  const int64_t bh = (int64_t)b * a.H + h;
  const float* base = a.w + b * a.ws[0] + h * a.ws[1];
  const int rpw = a.rc_rows / kRcWaves;  // rows per wave
  const int t_first = chunk * a.rc_rows + wave * rpw;
  const int t_end = min(t_first + rpw, a.T);

  float cm[NK][4], cq[NK][4];
#pragma unroll
  for (int j = 0; j < NK; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) cm[j][i] = cq[j][i] = 0.f;

  // Loads are straight-line code at clamped (always valid) addresses, masked after the load,
  // so the compiler can wait for exactly the row it consumes: with A % 4 == 0 every float4
  // column 4*(lane + 64 j) clamped to A - 4 lies inside the row.
  bool colv[NK][4];
  int colc[NK];
#pragma unroll
  for (int j = 0; j < NK; ++j) {
    const int col = 4 * (lane + 64 * j);
    colc[j] = min(col, a.A - 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) colv[j][i] = col + i < cap;
  }
  auto load_row = [&](int t, float (&x)[NK][4]) __attribute__((always_inline)) {
    const float* src = base + (int64_t)min(t, t_end - 1) * a.ws[2];
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      f32x4 v;
      if constexpr (NT) v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + colc[j]));
      else v = *reinterpret_cast<const f32x4*>(src + colc[j]);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[j][i] = v[i];
    }
  };

  int k = 0;  // valid rows folded in by this wave
  auto row_step = [&](int t, float (&x)[NK][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NK; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) x[j][i] = colv[j][i] ? x[j][i] : -INFINITY;
    // max(x) * log2e == max(x * log2e): the scaling is monotone, rounding included.
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NK; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, x[j][i]);
    float2 st;
    st.x = wave_max(mx) * kLog2e;
    // e = exp2(x*log2e - m) exactly as softmax_value forms it; kept for the column update
    // (-inf -> 0).
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < NK; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[j][i] = softmax_exp(x[j][i], st.x);
        sum += x[j][i];
      }
    st.y = 1.f / wave_sum(sum);
    if (lane == 0) a.rs[bh * a.T + t] = st;
    if (t < rows_valid) {
      ++k;
      const float inv = 1.f / (float)k;
#pragma unroll
      for (int j = 0; j < NK; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = softmax_scale_e(x[j][i], st.y);
          const float d = p - cm[j][i];
          cm[j][i] += d * inv;
          cq[j][i] += d * (p - cm[j][i]);
        }
    }
  };

  // Three rows in flight while a row is processed: four row buffers in rotation, eight rows
  // per unrolled iteration so each buffer keeps its role across iterations.
  constexpr int NB = 4;
  float xb[NB][NK][4];
  static_for<NB - 1>([&](int r) __attribute__((always_inline)) { load_row(t_first + r, xb[r]); });
  for (int t8 = t_first; t8 < t_end; t8 += 2 * NB) {
    static_for<2 * NB>([&](int r) __attribute__((always_inline)) {
      const int t = t8 + r;
      load_row(t + NB - 1, xb[(r + NB - 1) % NB]);
      if (t < t_end) row_step(t, xb[r % NB]);
    });
  }

  // Merge the waves' accumulators: 2+3 into 0+1, then 1 into 0.
  __shared__ f32x4 red[2][NK * 64][2];  // [wave slot][lane j][mean4 | M2 4]
  auto wave_rows = [&](int w) {
    const int lo = chunk * a.rc_rows + w * rpw;
    const int hi = min(lo + rpw, rows_valid);
    return (float)(hi > lo ? hi - lo : 0);
  };
  float n_self = (float)k;
#pragma unroll
  for (int step = 0; step < 2; ++step) {
    const int half = step == 0 ? 2 : 1;
    if (wave >= half && wave < 2 * half) {
#pragma unroll
      for (int j = 0; j < NK; ++j) {
        red[wave - half][j * 64 + lane][0] = f32x4{cm[j][0], cm[j][1], cm[j][2], cm[j][3]};
        red[wave - half][j * 64 + lane][1] = f32x4{cq[j][0], cq[j][1], cq[j][2], cq[j][3]};
      }
    }
    __syncthreads();
    if (wave < half) {
      float n_other = wave_rows(wave + half);
      if (step == 1) n_other += wave_rows(3);  // wave 1 already holds waves 1 and 3
#pragma unroll
      for (int j = 0; j < NK; ++j) {
        const f32x4 om = red[wave][j * 64 + lane][0];
        const f32x4 oq = red[wave][j * 64 + lane][1];
#pragma unroll
        for (int i = 0; i < 4; ++i) chan_merge(n_self, cm[j][i], cq[j][i], n_other, om[i], oq[i]);
      }
      n_self += n_other;
    }
    __syncthreads();
  }
  if (wave == 0 && n_self > 0.f) {
    const int n_chunks = (a.T + a.rc_rows - 1) / a.rc_rows;
    float2* part = a.part + (bh * n_chunks + chunk) * a.cpitch;
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const int col = 4 * (lane + 64 * j);
      if (col < cap) {
        // (mean, M2) pairs of 4 columns: 32 bytes.
        f32x4* dst = reinterpret_cast<f32x4*>(part + col);
        dst[0] = f32x4{cm[j][0], cq[j][0], cm[j][1], cq[j][1]};
        dst[1] = f32x4{cm[j][2], cq[j][2], cm[j][3], cq[j][3]};
      }
    }
  }
}

// Batch rows b < nt_b are read with nontemporal loads (streamed past the caches: 4.5 -> 5.3
// TB/s); the last ones normally, so that they are still in the 256 MB Infinity Cache when the
// filter pass, which starts from the last batch row, reads them again.
template <int NK>
__global__ __launch_bounds__(256) void dtw_rowcol_kernel(DtwArgs a) {
  const int chunk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  if (b < a.nt_b) rowcol_body<NK, true>(a, chunk, h, b);
  else rowcol_body<NK, false>(a, chunk, h, b);
}

// Final column statistics from the chunk partials: cs = (mean, 1/sqrt(max(var, 1e-12))) with
// mean and var dividing by lens[b] (which may exceed T: the reference divides by the length,
// dtw_align.py:731-736). One thread per column; grid (ceil(need / 256), H, B).
__global__ __launch_bounds__(256) void dtw_col_merge_kernel(DtwArgs a, int need) {
  const int b = blockIdx.z, h = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int cap = clamp_cap(a.caps[b], a.A);
  const int len = a.lens[b];
  if (cap <= 0 || len <= 0 || c >= cap || c >= need) return;
  const int rows_valid = len < a.T ? len : a.T;
  const int n_chunks = (a.T + a.rc_rows - 1) / a.rc_rows;
  const int64_t bh = (int64_t)b * a.H + h;
  const float2* part = a.part + bh * n_chunks * a.cpitch + c;
  float n = 0.f, mean = 0.f, m2 = 0.f;
  for (int i = 0; i * a.rc_rows < rows_valid; ++i) {
    const int rows_i = min(rows_valid - i * a.rc_rows, a.rc_rows);
    const float2 pi = part[(int64_t)i * a.cpitch];
    chan_merge(n, mean, m2, (float)rows_i, pi.x, pi.y);
    n += (float)rows_i;
  }
  float var;
  if (len == rows_valid) {
    var = m2 / (float)len;
  } else {  // rows beyond T count in the divisor only
    const float mean_len = mean * (n / (float)len);
    const float d = mean - mean_len;
    var = (m2 + n * d * d) / (float)len;
    mean = mean_len;
  }
  var = var < 1e-12f ? 1e-12f : var;
  float2 r;
  r.x = mean;
  r.y = 1.f / sqrtf(var);
  a.cs[bh * a.cpitch + c] = r;
}

// ---------------------------------------------------------------------------------------------
// Median selection. Every routine returns an element of the window, so the result equals the
// reference's sort / bubble-network median for finite inputs.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void cx(float& lo, float& hi) {
  const float a = fminf(lo, hi);
  hi = fmaxf(lo, hi);
  lo = a;
}

// Medians of the 4 width-7 windows over x[0..9] (window i = x[i..i+6]), 30 min/max operations
// instead of 4 separate networks. Windows (0,1) share x[1..6] and windows (2,3) share x[3..8];
// both share x[3..6]. With t = sorted x[3..6] and a <= b the pair's two extra shared values, the
// 3rd and 4th smallest of the 6 shared values are
//   s2 = min(t2, max(t1, a), max(t0, b)),  s3 = min(t3, max(t2, a), max(t1, b))
// (k-th smallest of a merge of two sorted lists), and the median of the shared 6 plus one more
// value v is med3(s2, v, s3). Checked against a sort on all 1024 0-1 inputs and on random inputs
// with ties.
__device__ __forceinline__ void median7_x4(const float (&x)[10], float (&out)[4]) {
  float t0 = x[3], t1 = x[4], t2 = x[5], t3 = x[6];
  cx(t0, t1); cx(t2, t3); cx(t0, t2); cx(t1, t3); cx(t1, t2);
  auto mid = [&](float a, float b, float& s2, float& s3) {
    cx(a, b);
    s2 = fminf(fminf(t2, fmaxf(t1, a)), fmaxf(t0, b));
    s3 = fminf(fminf(t3, fmaxf(t2, a)), fmaxf(t1, b));
  };
  float s2, s3;
  mid(x[1], x[2], s2, s3);
  out[0] = __builtin_amdgcn_fmed3f(s2, x[0], s3);
  out[1] = __builtin_amdgcn_fmed3f(s2, x[7], s3);
  mid(x[7], x[8], s2, s3);
  out[2] = __builtin_amdgcn_fmed3f(s2, x[2], s3);
  out[3] = __builtin_amdgcn_fmed3f(s2, x[9], s3);
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

// Medians of the 4 windows of width 2*PAD+1 over x[0 .. 3+2*PAD].
template <int PAD>
__device__ __forceinline__ void window_medians(const float (&x)[4 + 2 * PAD], float (&out)[4]) {
  if constexpr (PAD == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = x[i];
  } else if constexpr (PAD == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __builtin_amdgcn_fmed3f(x[i], x[i + 1], x[i + 2]);
  } else if constexpr (PAD == 3) {
    median7_x4(x, out);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[2 * PAD + 1];
#pragma unroll
      for (int j = 0; j < 2 * PAD + 1; ++j) v[j] = x[i + j];
      out[i] = median_generic<2 * PAD + 1>(v);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Normalise + median filter + head mean. Grid: (ceil(C / 64), ceil(T / 16), B), 256 threads.
// The LDS tile holds 16 rows x columns [c0 - 8, c0 + 72) of z; only the float4 columns that
// reach within PAD of the strip are filled. Load mapping: thread = (float4 column lq, row group
// lg), rows lg, lg + RG. Filter mapping: thread = (row tid/16, output columns 4*(tid%16) .. +3).
// ---------------------------------------------------------------------------------------------
template <int PAD>
__global__ __launch_bounds__(256) void dtw_filter_kernel(DtwArgs a) {
  constexpr int kQ0 = (kHalo - PAD) / 4;                   // first float4 column filled
  constexpr int kQ1 = (kHalo + kColBlock + PAD + 3) / 4;   // one past the last
  constexpr int NQ = kQ1 - kQ0;
  constexpr int RG = 256 / NQ;
  constexpr int RPT = (kFiltRows + RG - 1) / RG;
  const int b = blockIdx.z;
  const int t0 = blockIdx.y * kFiltRows;
  const int c0 = blockIdx.x * kColBlock;
  const int tid = threadIdx.x;
  const int cap = clamp_cap(a.caps[b], a.A);
  const int len = a.lens[b];

  const int fr = tid >> 4;        // filter row
  const int fq = 4 * (tid & 15);  // first of 4 output columns
  const int ot = t0 + fr;

  if (cap <= 0 || len <= 0) {  // 0/0 in the reference: the whole batch row is NaN
    if (ot < a.T)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c0 + fq + i < a.C) a.out[b * a.os[0] + (int64_t)ot * a.os[1] + c0 + fq + i] = __builtin_nanf("");
    return;
  }

  __shared__ f32x4 tile4[kFiltRows * kTilePitch / 4];
  __shared__ float2 rstat[kFiltRows];
  __shared__ f32x4 cstat[NQ][2];  // column (mean, 1/std) of the tile's float4 columns
  float* tile = reinterpret_cast<float*>(tile4);

  const int lq = tid % NQ, lg = tid / NQ;
  const bool lactive = lg < RG;
  const int gc = c0 - kHalo + 4 * (kQ0 + lq);  // first (unreflected) column of this thread's 4
  // Fast: 4 in-range valid columns, loaded with one 16-byte load from aligned rows.
  const bool fast = a.vec && gc >= 0 && gc + 4 <= cap;
  int gs[4];
  bool vs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int g = gc + i;
    // Only columns within +-PAD of an output column < C are read.
    const bool need = g >= c0 - PAD && g < c0 + kColBlock + PAD && g < a.C + PAD;
    if (g < 0) g = -g;
    if (g >= a.A) g = 2 * (a.A - 1) - g;
    gs[i] = g;
    vs[i] = lactive && need && g < cap;  // g >= cap: p = 0, mean 0, z = 0
  }
  const bool any_valid = vs[0] || vs[1] || vs[2] || vs[3];

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  // Everything one head needs from global memory: this thread's scores, and (for row group 0)
  // its columns' statistics, (for tid < 16) one row's statistics. Two heads are in flight.
  struct Prefetch {
    float x[RPT][4];
    f32x4 c[2];
    float2 r;
  };
  Prefetch pf[2];

  auto issue = [&](int h, Prefetch& q) {
    const int64_t bh = (int64_t)b * a.H + h;
    const float* src = a.w + b * a.ws[0] + h * a.ws[1];
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int t = t0 + lg + RG * r;
      const bool row_ok = lactive && lg + RG * r < kFiltRows && t < a.T;
      const float* rowp = src + (int64_t)t * a.ws[2];
      if (fast) {
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        if (row_ok) v = *reinterpret_cast<const f32x4*>(rowp + gc);
#pragma unroll
        for (int i = 0; i < 4; ++i) q.x[r][i] = v[i];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) q.x[r][i] = (row_ok && vs[i]) ? rowp[gs[i]] : 0.f;
      }
    }
    if (lg == 0) {  // one thread per float4 column fetches the statistics for all row groups
      const float2* cs = a.cs + bh * a.cpitch;
      if (fast) {
        q.c[0] = *reinterpret_cast<const f32x4*>(cs + gc);
        q.c[1] = *reinterpret_cast<const f32x4*>(cs + gc + 2);
      } else {
        float2 c[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c[i] = vs[i] ? cs[gs[i]] : make_float2(0.f, 0.f);
        q.c[0] = f32x4{c[0].x, c[0].y, c[1].x, c[1].y};
        q.c[1] = f32x4{c[2].x, c[2].y, c[3].x, c[3].y};
      }
    }
    if (tid < kFiltRows) {
      const int t = t0 + tid;
      q.r = t < a.T ? a.rs[bh * a.T + t] : make_float2(0.f, 0.f);
    }
  };

  auto head = [&](int h, Prefetch& q) {
    if (tid < kFiltRows) rstat[tid] = q.r;
    if (lg == 0) {
      cstat[lq][0] = q.c[0];
      cstat[lq][1] = q.c[1];
    }
    __syncthreads();
    // Normalised tile: z = (softmax - mean) / std; 0 in masked columns.
    if (lactive) {
      const f32x4 c01 = cstat[lq][0], c23 = cstat[lq][1];
      const float cmean[4] = {c01[0], c01[2], c23[0], c23[2]};
      const float crstd[4] = {c01[1], c01[3], c23[1], c23[3]};
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const int rr = lg + RG * r;
        if (rr < kFiltRows) {
          f32x4 z = f32x4{0.f, 0.f, 0.f, 0.f};
          if (any_valid) {
            const float2 st = rstat[rr];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (vs[i]) z[i] = (softmax_value(q.x[r][i], st) - cmean[i]) * crstd[i];
          }
          tile4[(rr * kTilePitch) / 4 + kQ0 + lq] = z;
        }
      }
    }
    __syncthreads();
    if (h + 2 < a.H) issue(h + 2, q);  // refill this slot; it lands two heads from now
    {
      // Window values: tile columns [fq + kHalo - PAD, fq + kHalo + 3 + PAD], read as float4s.
      constexpr int kJ0 = (kHalo - PAD) / 4, kJ1 = (kHalo + 3 + PAD) / 4;
      constexpr int kOff = kHalo - PAD - 4 * kJ0;
      float seg[4 * (kJ1 - kJ0 + 1)];
#pragma unroll
      for (int j = kJ0; j <= kJ1; ++j) {
        const f32x4 v = tile4[(fr * kTilePitch + fq) / 4 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i) seg[4 * (j - kJ0) + i] = v[i];
      }
      float win[4 + 2 * PAD];
#pragma unroll
      for (int i = 0; i < 4 + 2 * PAD; ++i) win[i] = seg[kOff + i];
      float med[4];
      window_medians<PAD>(win, med);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += med[i];
    }
    __syncthreads();  // the tile and the statistics are rewritten for the next head
  };

  issue(0, pf[0]);
  if (a.H > 1) issue(1, pf[1]);
  for (int h = 0; h < a.H; h += 2) {
    head(h, pf[0]);
    if (h + 1 < a.H) head(h + 1, pf[1]);
  }
  if (ot < a.T) {
    float* dst = a.out + b * a.os[0] + (int64_t)ot * a.os[1] + c0 + fq;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (c0 + fq + i < a.C) dst[i] = acc[i] / (float)a.H;
  }
}

// ---------------------------------------------------------------------------------------------
// Normalise + median filter + head mean over whole rows (rows 16-byte aligned, A % 4 == 0,
// A <= 2048): one workgroup per (4 rows, b), NT = 128 * ceil(A / 512) threads, one float4
// column each. Per head, the 4 rows are read as contiguous 16-byte vectors, normalised into an
// LDS tile with PAD reflected columns on each side, and each thread accumulates the medians of
// its 4 output columns in the 4 rows. Reading whole rows fetches every HBM line once.
//
// Latency: two heads' loads are in flight while a head is filtered. The loads are
// straight-line code at clamped (always valid) addresses, with out-of-range data masked after
// the load, so the compiler waits for exactly the head it consumes.
// ---------------------------------------------------------------------------------------------
constexpr int kBandRows = 4;
constexpr int kBandMaxA4 = 512;    // float4 columns per row (A <= 2048)
constexpr int kBandMaxHeads = 16;  // heads per call on this path (large-v3 aligns on 10)

template <int PAD, int NT>
__global__ __launch_bounds__(NT) void dtw_band_kernel(DtwArgs a) {
  // Last batch row first: the statistics pass ended there, so its scores are the ones still
  // held in the device-wide (infinity) cache.
  const int b = a.B - 1 - (int)blockIdx.y;
  const int t0 = (gridDim.x - 1 - blockIdx.x) * kBandRows;
  const int tid = threadIdx.x;
  const int cap = clamp_cap(a.caps[b], a.A);
  const int len = a.lens[b];
  const int A4 = a.A >> 2;
  const int n_rows = min(kBandRows, a.T - t0);

  if (cap <= 0 || len <= 0) {  // 0/0 in the reference: the whole batch row is NaN
    for (int r = 0; r < n_rows; ++r)
      for (int c = tid; c < a.C; c += NT) a.out[b * a.os[0] + (int64_t)(t0 + r) * a.os[1] + c] = __builtin_nanf("");
    return;
  }

  constexpr int kBandPitch = 4 * NT + 16;  // floats: 8 halo columns each side
  __shared__ f32x4 tile4[kBandRows * kBandPitch / 4];
  float* tile = reinterpret_cast<float*>(tile4);

  const bool active = tid < A4;
  const int col = 4 * (active ? tid : A4 - 1);  // clamped: every load address is valid
  bool valid[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) valid[i] = active && col + i < cap;

  struct Prefetch {
    f32x4 x[kBandRows];
    f32x4 c[2];  // (mean, 1/std) of the 4 columns
    float2 r[kBandRows];
  };
  Prefetch pf[2];

  auto issue = [&](int h, Prefetch& q) __attribute__((always_inline)) {
    h = min(h, a.H - 1);
    const int64_t bh = (int64_t)b * a.H + h;
    const float* src = a.w + b * a.ws[0] + h * a.ws[1];
    const float2* cs = a.cs + bh * a.cpitch + col;
    q.c[0] = *reinterpret_cast<const f32x4*>(cs);
    q.c[1] = *reinterpret_cast<const f32x4*>(cs + 2);
#pragma unroll
    for (int r = 0; r < kBandRows; ++r) {
      const int t = min(t0 + r, a.T - 1);
      q.r[r] = a.rs[bh * a.T + t];
      q.x[r] = *reinterpret_cast<const f32x4*>(src + (int64_t)t * a.ws[2] + col);
    }
  };

  float acc[kBandRows][4];
#pragma unroll
  for (int r = 0; r < kBandRows; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[r][i] = 0.f;

  auto head = [&](int h, Prefetch& q) __attribute__((always_inline)) {
    // Normalised rows: z = (softmax - mean) / std; 0 in masked columns (c >= cap). Columns
    // 1..PAD and A-1-PAD..A-2 are also written to their reflected positions -1..-PAD and
    // A..A-1+PAD (torch's reflect padding).
    const float cmean[4] = {q.c[0][0], q.c[0][2], q.c[1][0], q.c[1][2]};
    const float crstd[4] = {q.c[0][1], q.c[0][3], q.c[1][1], q.c[1][3]};
#pragma unroll
    for (int r = 0; r < kBandRows; ++r) {
      f32x4 z;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = (softmax_value(q.x[r][i], q.r[r]) - cmean[i]) * crstd[i];
        z[i] = valid[i] ? v : 0.f;
      }
      if (active) {
        tile4[(r * kBandPitch + kHalo) / 4 + tid] = z;
        if constexpr (PAD > 0) {
          float* row = tile + r * kBandPitch + kHalo;
          if (col <= PAD) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (col + i >= 1 && col + i <= PAD) row[-(col + i)] = z[i];
          }
          if (col + 3 >= a.A - 1 - PAD) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int c = col + i;
              if (c >= a.A - 1 - PAD && c <= a.A - 2) row[2 * (a.A - 1) - c] = z[i];
            }
          }
        }
      }
    }
    __syncthreads();
    const bool live = h < a.H;  // a padding head (odd H) is computed but not accumulated
    issue(h + 2, q);            // refill this slot; it is consumed two heads from now
    {
      constexpr int kJ0 = (kHalo - PAD) / 4, kJ1 = (kHalo + 3 + PAD) / 4;
      constexpr int kOff = kHalo - PAD - 4 * kJ0;
#pragma unroll
      for (int r = 0; r < kBandRows; ++r) {
        float seg[4 * (kJ1 - kJ0 + 1)];
#pragma unroll
        for (int j = kJ0; j <= kJ1; ++j) {
          const f32x4 v = tile4[(r * kBandPitch) / 4 + tid + j];
#pragma unroll
          for (int i = 0; i < 4; ++i) seg[4 * (j - kJ0) + i] = v[i];
        }
        float win[4 + 2 * PAD];
#pragma unroll
        for (int i = 0; i < 4 + 2 * PAD; ++i) win[i] = seg[kOff + i];
        float med[4];
        window_medians<PAD>(win, med);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][i] += live ? med[i] : 0.f;
      }
    }
    __syncthreads();  // the tile is rewritten for the next head
  };

  issue(0, pf[0]);
  issue(1, pf[1]);
  for (int h = 0; h < a.H; h += 2) {
    head(h, pf[0]);
    head(h + 1, pf[1]);
  }
  if (tid < ((a.C + 3) >> 2)) {
#pragma unroll
    for (int r = 0; r < kBandRows; ++r) {
      if (r < n_rows) {
        float* dst = a.out + b * a.os[0] + (int64_t)(t0 + r) * a.os[1] + 4 * tid;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * tid + i < a.C) dst[i] = acc[r][i] / (float)a.H;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Width-7 normalise + median + head mean, one wavefront per (b, 4 rows, 250-column segment).
// Lane L holds columns s0 - 3 + 4L .. +3 of each row (the segment's 250 output columns plus
// 3 on each side), so every window lies inside its own wavefront's strip: the strip goes
// through a wavefront-private LDS row and no workgroup barrier is needed. Every lane reads
// its 4 columns with one 16-byte load (4-byte aligned) at an address clamped into the row;
// in the first and last segment the lanes whose columns leave the row then take their values
// from the strip at the reflected columns (torch's reflect padding), one LDS gather per row.
// ---------------------------------------------------------------------------------------------
constexpr int kSegOut = 250;
constexpr int kSegRows = 4;  // rows per wavefront (2, 6 and 8 measured slower)
constexpr int kSegPf = 2;    // heads in flight per wavefront (3 measured slower)
constexpr int kSegWaves = 4;  // independent wavefronts per workgroup (1, 2 and 8 measured slower)
constexpr int kSegPitch = 272;  // floats per strip row (256 written + the last lanes' overrun)
typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));

__global__ __launch_bounds__(kSegWaves * 64) void dtw_seg_kernel(DtwArgs a, int n_seg) {
  __shared__ f32x4 strips[kSegWaves][kSegRows * kSegPitch / 4];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar indexing
  const int n_rg = (a.T + kSegRows - 1) / kSegRows;
  const int item = blockIdx.x * kSegWaves + w;
  if (item >= a.B * n_rg * n_seg) return;  // whole wavefronts; no barriers below
  const int seg = item % n_seg;
  const int rest = item / n_seg;
  const int t0 = (rest % n_rg) * kSegRows;
  const int b = a.B - 1 - rest / n_rg;  // last batch row first: the statistics pass ended there
  const int s0 = seg * kSegOut;
  const int n_rows = min(kSegRows, a.T - t0);
  const int cap = clamp_cap(a.caps[b], a.A);
  const int len = a.lens[b];
  const int n_out = min(kSegOut, a.C - s0);
  const int oc = 4 * lane;
  float* dst = a.out + b * a.os[0] + (int64_t)t0 * a.os[1] + s0 + oc;
  if (cap <= 0 || len <= 0) {  // 0/0 in the reference: the whole batch row is NaN
    for (int r = 0; r < n_rows; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (oc + i < n_out) dst[r * a.os[1] + i] = __builtin_nanf("");
    return;
  }
  f32x4* const strip = strips[w];
  const int sb = s0 - 3;                             // column of strip slot 0
  const int lc = min(max(sb + 4 * lane, 0), a.A - 4);  // first column this lane loads
  const bool edge = sb < 0 || sb + 4 * 64 > a.A;       // wave-uniform
  bool valid[4];
  int src[4];  // edge segments: the strip slot holding the reflected column of slot 4L + i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    valid[i] = lc + i < cap;
    int c = sb + 4 * lane + i;
    c = c < 0 ? -c : c;
    c = c > a.A - 1 ? 2 * (a.A - 1) - c : c;
    c = min(max(c, 0), a.A - 1);
    const int owner = (c - sb) >> 2;
    src[i] = 4 * owner + c - min(max(sb + 4 * owner, 0), a.A - 4);
  }

  struct Prefetch {
    f32x4u x[kSegRows];
    f32x4u c[2];  // (mean, 1/std) of the 4 columns
    float2 r[kSegRows];
  };
  Prefetch pf[kSegPf];
  auto issue = [&](int h, Prefetch& q) __attribute__((always_inline)) {
    h = min(h, a.H - 1);
    const int64_t bh = (int64_t)b * a.H + h;
    const float* rows = a.w + b * a.ws[0] + h * a.ws[1];
    const float2* cs = a.cs + bh * a.cpitch + lc;
    q.c[0] = *reinterpret_cast<const f32x4u*>(cs);
    q.c[1] = *reinterpret_cast<const f32x4u*>(cs + 2);
#pragma unroll
    for (int r = 0; r < kSegRows; ++r) {
      const int t = min(t0 + r, a.T - 1);
      q.r[r] = a.rs[bh * a.T + t];
      q.x[r] = *reinterpret_cast<const f32x4u*>(rows + (int64_t)t * a.ws[2] + lc);
    }
  };
  float acc[kSegRows][4];
#pragma unroll
  for (int r = 0; r < kSegRows; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[r][i] = 0.f;

  auto head = [&](Prefetch& q, int h_next) __attribute__((always_inline)) {
    const float cmean[4] = {q.c[0][0], q.c[0][2], q.c[1][0], q.c[1][2]};
    const float crstd[4] = {q.c[0][1], q.c[0][3], q.c[1][1], q.c[1][3]};
#pragma unroll
    for (int r = 0; r < kSegRows; ++r) {
      f32x4 z;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = (softmax_value(q.x[r][i], q.r[r]) - cmean[i]) * crstd[i];
        z[i] = valid[i] ? v : 0.f;
      }
      strip[r * (kSegPitch / 4) + lane] = z;
    }
    issue(h_next, q);  // refill this slot
    // The strip rows are written and read by this wavefront's own lanes: LDS executes one
    // wavefront's instructions in order, so only the compiler must not reorder them.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (edge) {
      const float* sf = reinterpret_cast<const float*>(strip);
      f32x4 g[kSegRows];
#pragma unroll
      for (int r = 0; r < kSegRows; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) g[r][i] = sf[r * kSegPitch + src[i]];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
      for (int r = 0; r < kSegRows; ++r) strip[r * (kSegPitch / 4) + lane] = g[r];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
#pragma unroll
    for (int r = 0; r < kSegRows; ++r) {
      float win[12];
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const f32x4 v = strip[r * (kSegPitch / 4) + lane + j];
#pragma unroll
        for (int i = 0; i < 4; ++i) win[4 * j + i] = v[i];
      }
      float x10[10];
#pragma unroll
      for (int i = 0; i < 10; ++i) x10[i] = win[i];
      float med[4];
      median7_x4(x10, med);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[r][i] += med[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  };
  static_for<kSegPf>([&](int i) __attribute__((always_inline)) { issue(i, pf[i]); });
  // Whisper's shape fully unrolled: with no loop-carried load registers each wait covers
  // exactly the head it consumes.
  static_for<kBandMaxHeads>([&](int h) __attribute__((always_inline)) {
    if (h < a.H) head(pf[h % kSegPf], h + kSegPf);
  });
#pragma unroll
  for (int r = 0; r < kSegRows; ++r) {
    if (r < n_rows) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (oc + i < n_out) dst[r * a.os[1] + i] = acc[r][i] / (float)a.H;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Fused path: the scores S = (Q_h K_h^T) * s^2 of the alignment heads are computed on the matrix
// cores inside both passes (CrossAttnCapture.compute_attention, dtw_align.py:553-586, then
// _dtw_prep_batch), so the [B, H, T, A] fp32 tensor is never written or read.
//
// One 16 x 16 score tile = two v_mfma_f32_16x16x32 over the 64 head dimensions; both passes
// call qk_product with the same operands, so every score is bit-identical between them (the exact
// zero of a zero-variance column depends on it). The products stay unscaled: s^2 is folded,
// with log2e, into the softmax's FMA (softmax_exp_c). Lane l: text row 4*(l/16) + i of the tile
// (i = 0..3), key l % 16; operands are 16-byte slices of the head rows (dims 8*(l/16) and
// 32 + 8*(l/16)).
// ---------------------------------------------------------------------------------------------
template <typename T> struct QkMfma;
template <> struct QkMfma<Bf16> {
  typedef bf16x8 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct QkMfma<F16> {
  typedef f16x8 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ void qk_row_ops(const DtwQkArgs& q, int h, int b, int t,
                                           typename QkMfma<T>::op_t (&qa)[2]) {
  typedef typename QkMfma<T>::op_t op_t;
  const int kh = 8 * ((threadIdx.x & 63) >> 4);
  const char* row = static_cast<const char*>(q.q[h]) + (b * q.qs[0] + (int64_t)t * q.qs[1]) * 2;
  qa[0] = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(row + kh * 2));
  qa[1] = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(row + (32 + kh) * 2));
}

template <typename T> struct QkKey {
  typename QkMfma<T>::op_t k0, k1;
};

template <typename T>
__device__ __forceinline__ QkKey<T> qk_key_ops(const DtwQkArgs& q, int h, int b, int key) {
  typedef typename QkMfma<T>::op_t op_t;
  const int kh = 8 * ((threadIdx.x & 63) >> 4);
  // a wave-uniform base and a 32-bit per-lane offset (one batch row of keys is < 4 GiB)
  const char* base = static_cast<const char*>(q.k[h]) + b * q.ks[0] * 2;
  const char* row = base + (uint32_t)(key * (uint32_t)q.ks[1] * 2u);
  QkKey<T> k;
  k.k0 = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(row + kh * 2));
  k.k1 = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(row + (32 + kh) * 2));
  return k;
}

template <typename T>
__device__ __forceinline__ f32x4 qk_product(const DtwQkArgs& q, const QkKey<T>& k,
                                            const typename QkMfma<T>::op_t (&qa)[2]) {
  (void)q;
  f32x4 acc = QkMfma<T>::run(qa[0], k.k0, f32x4{0.f, 0.f, 0.f, 0.f});
  return QkMfma<T>::run(qa[1], k.k1, acc);  // unscaled: the softmax applies scale^2 * log2e
}

// max / sum over the 16 lanes of a lane group (one DPP row), every lane gets the result
__device__ __forceinline__ float group16_max(float v) {
  v = fmaxf(v, dpp_xor1(v));
  v = fmaxf(v, dpp_xor2(v));
  v = fmaxf(v, dpp_half_mirror(v));
  return fmaxf(v, dpp_row_mirror(v));
}
// sum over lanes l, l^16, l^32, l^48 (the four lane groups), every lane gets the result
__device__ __forceinline__ float groups4_sum(float v) {
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
}

// Chan's merge of the Welford states (n, mean, M2) held by lanes l and l ^ 32 (X = 32) or by the
// two 16-lane rows of a pair (X = 16); every lane of the pair gets the same merged state.
template <int X>
__device__ __forceinline__ void lane_pair_merge(float& n, float& mean, float& m2) {
  auto swap = [](float v) {
    if constexpr (X == 32)
      return __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    else
      return __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  };
  const auto rn = swap(n), rm = swap(mean), rq = swap(m2);
  float na = __uint_as_float(rn[0]), ma = __uint_as_float(rm[0]), qa = __uint_as_float(rq[0]);
  chan_merge(na, ma, qa, __uint_as_float(rn[1]), __uint_as_float(rm[1]), __uint_as_float(rq[1]));
  n = na + __uint_as_float(rn[1]);
  mean = ma;
  m2 = qa;
}

constexpr int kQkWaves = 8;
constexpr int kQkTilesPerWave = 12;  // 8 wavefronts x 12 tiles x 16 keys = 1536 >= A

// Row statistics and column Welford partials of one (row chunk, h, b) from Q / K: 16 text rows
// at a time, the 8 wavefronts splitting the key tiles (tile j on wavefront j % 8). Row max and
// sum: within a lane, across its lane group (DPP), across the wavefronts (LDS). Column states:
// each lane keeps a running Welford state of its key column over the rows its lane group holds
// (rows 4*grp .. 4*grp + 3 of every block), folded in 4 rows at a time; the four lane groups'
// states are merged once, at the end of the chunk.
template <typename T>
__global__ __launch_bounds__(512) void dtw_qk_rowcol_kernel(DtwArgs a, DtwQkArgs q) {
  typedef typename QkMfma<T>::op_t op_t;
  // logical order: chunks fastest, then h, then b; remapped so that the chunks of one head run
  // on one XCD and read its keys through the same L2
  const int n_chunks = (a.T + a.rc_rows - 1) / a.rc_rows;
  const int w = remap_xcd(blockIdx.x, gridDim.x);
  const int chunk = w % n_chunks, h = (w / n_chunks) % a.H, b = w / (n_chunks * a.H);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane >> 4;
  const int cap = clamp_cap(a.caps[b], a.A);
  const int len = a.lens[b];
  if (cap <= 0 || len <= 0) return;  // the filter writes NaN for this batch row
  const int rows_valid = len < a.T ? len : a.T;
  const int64_t bh = (int64_t)b * a.H + h;
  const int n_tiles = (a.A + 15) >> 4;
  const float csc = q.scale2 * kLog2e;  // the same value in the filter pass

  // this wavefront's key operands, the same for every row block of the chunk: held in registers
  QkKey<T> kop[kQkTilesPerWave];
#pragma unroll
  for (int u = 0; u < kQkTilesPerWave; ++u)
    kop[u] = qk_key_ops<T>(q, h, b, min(16 * (wave + kQkWaves * u) + (lane & 15), a.A - 1));

  __shared__ float red[2][kQkWaves][16];  // per-wavefront row max / row sum
  float mu[kQkTilesPerWave], m2[kQkTilesPerWave];
#pragma unroll
  for (int u = 0; u < kQkTilesPerWave; ++u) mu[u] = m2[u] = 0.f;
  float n_l = 0.f;  // valid rows folded into this lane's states

  const int t_lo = chunk * a.rc_rows;
  const int t_hi = min(t_lo + a.rc_rows, a.T);
  op_t qn[2];  // the query rows of the next block, loaded one block ahead
  qk_row_ops<T>(q, h, b, min(t_lo + (lane & 15), a.T - 1), qn);
  for (int t0 = t_lo; t0 < t_hi; t0 += 16) {
    op_t qa[2] = {qn[0], qn[1]};
    if (t0 + 16 < t_hi) qk_row_ops<T>(q, h, b, min(t0 + 16 + (lane & 15), a.T - 1), qn);
    float s[kQkTilesPerWave][4];
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int u = 0; u < kQkTilesPerWave; ++u) {
      const int j = wave + kQkWaves * u;
      const int key = 16 * j + (lane & 15);
      const f32x4 acc = qk_product<T>(q, kop[u], qa);
      const bool ok = j < n_tiles && key < cap;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[u][i] = ok ? acc[i] : -INFINITY;
        mx[i] = fmaxf(mx[i], s[u][i]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) mx[i] = group16_max(mx[i]);
    if ((lane & 15) == 0)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[0][wave][4 * grp + i] = mx[i];
    __syncthreads();
    float2 st[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * grp + i;
      float m = red[0][0][r];
#pragma unroll
      for (int w = 1; w < kQkWaves; ++w) m = fmaxf(m, red[0][w][r]);
      st[i].x = m * csc;  // max(x) * c is max(x * c) exactly: c > 0 and rounding is monotone
    }
    float sm[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kQkTilesPerWave; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[u][i] = softmax_exp_c(s[u][i], csc, st[i].x);  // -inf -> 0
        sm[i] += s[u][i];
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) sm[i] = group_sum<16>(sm[i]);
    if ((lane & 15) == 0)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[1][wave][4 * grp + i] = sm[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * grp + i;
      float t = red[1][0][r];
#pragma unroll
      for (int w = 1; w < kQkWaves; ++w) t += red[1][w][r];
      st[i].y = 1.f / t;
    }
    if (wave == 0)  // lane i of lane group grp stores row 4*grp + i
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if ((lane & 15) == i && t0 + 4 * grp + i < a.T) a.rs[bh * a.T + t0 + 4 * grp + i] = st[i];
    if (t0 < rows_valid) {
      // fold this lane group's valid rows of the block (0..4 of them) into its column states
      bool rv[4];
      float fnb = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rv[i] = t0 + 4 * grp + i < rows_valid;
        fnb += rv[i] ? 1.f : 0.f;
      }
      const float n_new = n_l + fnb;
      const bool any = fnb > 0.f;
      const float inv_nb = any ? 1.f / fnb : 0.f;
      const float ra = any ? fnb / n_new : 0.f;
      const float rb = any ? n_l * fnb / n_new : 0.f;
      // FULL: every row of the block is valid (all but the last block of a row range), so the
      // per-row selects drop out; the arithmetic is the same either way.
      auto fold = [&](auto full) __attribute__((always_inline)) {
        constexpr bool FULL = decltype(full)::value;
#pragma unroll
        for (int u = 0; u < kQkTilesPerWave; ++u) {
          float p[4], sum = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            p[i] = softmax_scale_e(s[u][i], st[i].y);
            sum += (FULL || rv[i]) ? p[i] : 0.f;
          }
          const float mean_b = sum * inv_nb;
          float sq = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float d = p[i] - mean_b;
            sq += (FULL || rv[i]) ? d * d : 0.f;
          }
          const float d = mean_b - mu[u];
          mu[u] += d * ra;
          m2[u] += sq + d * d * rb;
        }
      };
      if (t0 + 16 <= rows_valid) fold(std::true_type{});
      else fold(std::false_type{});
      n_l = n_new;
    }
  }
  // the chunk's partial (mean, M2) of every valid column, for dtw_col_merge_kernel
  if (t_lo < rows_valid) {
    float2* part = a.part + (bh * n_chunks + chunk) * a.cpitch;
#pragma unroll
    for (int u = 0; u < kQkTilesPerWave; ++u) {
      float n = n_l;
      lane_pair_merge<32>(n, mu[u], m2[u]);
      lane_pair_merge<16>(n, mu[u], m2[u]);
      const int c = 16 * (wave + kQkWaves * u) + (lane & 15);
      if (grp == 0 && c < cap) part[c] = make_float2(mu[u], m2[u]);
    }
  }
}

// Normalise + median filter + head mean from Q / K. One workgroup per (256 output columns,
// 32 text rows, b), 4 wavefronts. Per head the scores of the 32 rows over the segment and one
// 16-key tile of halo on each side are recomputed (key tile j on wavefront j % 4, both 16-row
// halves from one load of its key operands), normalised into an LDS tile [32][292] (reflected
// halo at the ends of the audio axis), and each lane accumulates the medians of one group of 4
// columns in 8 rows. The [B, H, T, A] scores are never stored; each WG reads 18 x 2 KB of K per
// head.
constexpr int kQsRows = 32;
constexpr int kQsSeg = 256;
constexpr int kQsKeyTiles = kQsSeg / 16 + 2;
constexpr int kQsPitch = kQsSeg + 32 + 4;  // 16-byte rows; the 4 lane groups' rows on distinct banks
constexpr int kQsTilesPerWave = (kQsKeyTiles + 3) / 4;

template <typename T, int PAD>
__global__ __launch_bounds__(256, 2) void dtw_qk_band_kernel(DtwArgs a, DtwQkArgs q) {
  typedef typename QkMfma<T>::op_t op_t;
  const int n_seg = (a.C + kQsSeg - 1) / kQsSeg, n_tb = (a.T + kQsRows - 1) / kQsRows;
  // logical order: row blocks fastest, then segments, then b; remapped so that the work items
  // reading one batch row's keys run on one XCD
  const int w = remap_xcd(blockIdx.x, gridDim.x);
  const int tb = w % n_tb, sg = (w / n_tb) % n_seg, b = w / (n_tb * n_seg);
  const int c0 = sg * kQsSeg, t0 = tb * kQsRows;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = lane >> 4;
  const int cap = clamp_cap(a.caps[b], a.A);
  const int len = a.lens[b];
  const int n_rows = min(kQsRows, a.T - t0);
  float* out = a.out + b * a.os[0];
  if (cap <= 0 || len <= 0) {  // 0/0 in the reference: the whole batch row is NaN
    for (int r = wave; r < n_rows; r += 4)
      for (int c = c0 + lane; c < min(c0 + kQsSeg, a.C); c += 64) out[(int64_t)(t0 + r) * a.os[1] + c] = __builtin_nanf("");
    return;
  }
  // double-buffered: head h is normalised into buffer h % 2, so the writes of head h + 1 never
  // meet the median reads of head h and one barrier per head suffices
  __shared__ __align__(16) float tiles[2][kQsRows * kQsPitch];
  const float csc = q.scale2 * kLog2e;  // the same value in the statistics pass
  const int key_base = c0 - 16;  // key of tile column 0

  float acc[kQsRows / 4][4];
#pragma unroll
  for (int k = 0; k < kQsRows / 4; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[k][i] = 0.f;

  // Operands of one head (query rows and row statistics of both halves, key operands and
  // column statistics of this wavefront's key tiles), loaded one head ahead: the loads of head
  // h + 1 are in flight during the median phase of head h.
  struct HeadOps {
    op_t qa[2][2];
    float2 st[2][4];
    QkKey<T> k[kQsTilesPerWave];
    float2 c[kQsTilesPerWave];
  };
  auto load = [&](int h, HeadOps& o) __attribute__((always_inline)) {
    const int64_t bh = (int64_t)b * a.H + h;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      qk_row_ops<T>(q, h, b, min(t0 + 16 * hf + (lane & 15), a.T - 1), o.qa[hf]);
#pragma unroll
      for (int i = 0; i < 4; ++i) o.st[hf][i] = a.rs[bh * a.T + min(t0 + 16 * hf + 4 * grp + i, a.T - 1)];
    }
    const float2* cs = a.cs + bh * a.cpitch;
#pragma unroll
    for (int i = 0; i < kQsTilesPerWave; ++i) {
      const int key = key_base + 16 * (wave + 4 * i) + (lane & 15);
      const int kc = key < 0 ? 0 : (key > a.A - 1 ? a.A - 1 : key);  // a valid address; unused if clamped
      if (wave + 4 * i < kQsKeyTiles) {
        o.k[i] = qk_key_ops<T>(q, h, b, kc);
        o.c[i] = cs[kc];
      }
    }
  };
  HeadOps cur;
  load(0, cur);
  for (int h = 0; h < a.H; ++h) {
    float* tile = tiles[h & 1];
    const f32x4* tile4 = reinterpret_cast<const f32x4*>(tile);
    f32x4 sc_all[kQsTilesPerWave][2];  // every tile's products first: the matrix-core latency overlaps
#pragma unroll
    for (int i = 0; i < kQsTilesPerWave; ++i)
      if (wave + 4 * i < kQsKeyTiles)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) sc_all[i][hf] = qk_product<T>(q, cur.k[i], cur.qa[hf]);
#pragma unroll
    for (int i = 0; i < kQsTilesPerWave; ++i) {
      const int j = wave + 4 * i;  // key tile
      if (j >= kQsKeyTiles) continue;
      const int key = key_base + 16 * j + (lane & 15);
      const bool ok = key >= 0 && key < cap;
      const float2 c = cur.c[i];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        float z[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // computed for every lane (a clamped key has a finite score), then selected: no branch
          const float v = (softmax_value_c(sc_all[i][hf][r], csc, cur.st[hf][r]) - c.x) * c.y;
          z[r] = ok ? v : 0.f;
        }
        float* row0 = tile + (16 * hf + 4 * grp) * kQsPitch;
        if (key >= 0 && key < a.A) {
#pragma unroll
          for (int r = 0; r < 4; ++r) row0[r * kQsPitch + key - key_base] = z[r];
        }
        if constexpr (PAD > 0) {
          // mirrored copies about column 0 and column A-1; only the tiles at the two ends of
          // the audio axis hold such keys (a wave-uniform test)
          const int k0 = key_base + 16 * j;
          if ((c0 == 0 && k0 <= PAD) || (k0 + 15 >= a.A - 1 - PAD && k0 <= a.A - 2)) {
            // on a short axis (A <= 2 * PAD + 1) one key can have both mirror images
            if (c0 == 0 && key >= 1 && key <= PAD) {
#pragma unroll
              for (int r = 0; r < 4; ++r) row0[r * kQsPitch + 16 - key] = z[r];
            }
            const int xr = 2 * (a.A - 1) - key - key_base;
            if (key >= a.A - 1 - PAD && key <= a.A - 2 && xr < kQsSeg + 32) {
#pragma unroll
              for (int r = 0; r < 4; ++r) row0[r * kQsPitch + xr] = z[r];
            }
          }
        }
      }
    }
    __syncthreads();
    if (h + 1 < a.H) load(h + 1, cur);  // cur is consumed: refill it for the next head
    {
      constexpr int kJ0 = (16 - PAD) / 4, kJ1 = (16 + 3 + PAD) / 4;
      constexpr int kOff = 16 - PAD - 4 * kJ0;
      constexpr int NJ = kJ1 - kJ0 + 1;
      // rows 4k + wave; the next row's reads are issued before this row's medians
      f32x4 segv[2][NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) segv[0][j] = tile4[(wave * kQsPitch) / 4 + lane + kJ0 + j];
#pragma unroll
      for (int k = 0; k < kQsRows / 4; ++k) {
        if (k + 1 < kQsRows / 4) {
          const int rn = 4 * (k + 1) + wave;
#pragma unroll
          for (int j = 0; j < NJ; ++j) segv[(k + 1) & 1][j] = tile4[(rn * kQsPitch) / 4 + lane + kJ0 + j];
        }
        float win[4 + 2 * PAD];
#pragma unroll
        for (int i = 0; i < 4 + 2 * PAD; ++i) win[i] = segv[k & 1][(kOff + i) / 4][(kOff + i) % 4];
        float med[4];
        window_medians<PAD>(win, med);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[k][i] += med[i];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kQsRows / 4; ++k) {
    const int r = 4 * k + wave;
    if (r < n_rows) {
      float* dst = out + (int64_t)(t0 + r) * a.os[1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = c0 + 4 * lane + i;
        if (c < a.C) dst[c] = acc[k][i] / (float)a.H;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Standalone median filter along the last axis (median_filter, dtw_align.py:156-167, and its
// sort-based form at dtw_align.py:65-78): width 2*PAD+1, reflect padding. One workgroup per
// row (per 2048-column piece of longer rows), 4 columns per lane: the columns and an 8-wide
// reflected halo go to LDS (16-byte loads when rows are 16-byte aligned), each lane takes the
// medians of 4 adjacent windows with the networks the prep's filter pass uses.
// ---------------------------------------------------------------------------------------------
constexpr int kMfMaxThreads = 512;  // 4 columns per lane: up to 2048 columns per workgroup

template <int PAD>
__global__ __launch_bounds__(kMfMaxThreads) void median_filter_kernel(MedianArgs a) {
  __shared__ __align__(16) float row[4 * kMfMaxThreads + 2 * kHalo];
  const int cols = 4 * blockDim.x;
  const int n_pieces = (a.N + cols - 1) / cols;
  const int c0 = (int)(blockIdx.x % n_pieces) * cols;
  const int64_t r = blockIdx.x / n_pieces;
  const float* src = a.x + r * a.xs;
  if (a.vec) {
    // interior as 16-byte loads (c0 and the row start are multiples of 4 floats), halo scalar
    for (int i = threadIdx.x; i < cols / 4; i += blockDim.x) {
      const int c = c0 + 4 * i;
      f32x4 v;
      if (c + 4 <= a.N) {
        v = *reinterpret_cast<const f32x4*>(src + c);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          int cc = c + j;
          cc = cc >= a.N ? 2 * (a.N - 1) - cc : cc;
          v[j] = src[cc < 0 ? 0 : cc];
        }
      }
      *reinterpret_cast<f32x4*>(&row[kHalo + 4 * i]) = v;
    }
    for (int i = threadIdx.x; i < 2 * kHalo; i += blockDim.x) {
      const int li = i < kHalo ? i : cols + i;  // left halo, then right halo
      int c = c0 - kHalo + li;
      c = c < 0 ? -c : (c >= a.N ? 2 * (a.N - 1) - c : c);
      c = c < 0 ? 0 : (c >= a.N ? a.N - 1 : c);
      row[li] = src[c];
    }
  } else {
    for (int i = threadIdx.x; i < cols + 2 * kHalo; i += blockDim.x) {
      int c = c0 - kHalo + i;
      c = c < 0 ? -c : (c >= a.N ? 2 * (a.N - 1) - c : c);  // reflect (N > PAD: in range for the halo used)
      c = c < 0 ? 0 : (c >= a.N ? a.N - 1 : c);               // columns no output reads: any valid address
      row[i] = src[c];
    }
  }
  __syncthreads();
  const int col = c0 + 4 * threadIdx.x;
  if (col >= a.N) return;
  float win[4 + 2 * PAD];
#pragma unroll
  for (int i = 0; i < 4 + 2 * PAD; ++i) win[i] = row[kHalo + 4 * threadIdx.x - PAD + i];
  float med[4];
  window_medians<PAD>(win, med);
  float* dst = a.y + r * a.ys;
  if (a.vec && col + 4 <= a.N) {
    __builtin_nontemporal_store(f32x4{med[0], med[1], med[2], med[3]}, reinterpret_cast<f32x4*>(dst + col));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (col + i < a.N) dst[col + i] = med[i];
  }
}

}  // namespace

// Workspace: row statistics [B*H*T], column statistics [B*H, cpitch], chunk partials
// [B*H, n_chunks, cpitch] (float2 each; cpitch = A rounded up to 4), each 256-byte aligned.
namespace {
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
}  // namespace

// Rows per chunk of the fused statistics pass (a multiple of the 4 waves), from sizes only.
int dtw_chunk_rows(int64_t B, int64_t H, int64_t T, int slots = kRcSlots) {
  int64_t n_chunks = slots / (B * H);
  if (n_chunks < 1) n_chunks = 1;
  int64_t rows = (T + n_chunks - 1) / n_chunks;
  rows = (rows + kRcWaves - 1) / kRcWaves * kRcWaves;
  return (int)(rows < kRcWaves ? kRcWaves : rows);
}

size_t dtw_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A) {
  const int64_t cpitch = (A + 3) & ~int64_t(3);
  const int64_t rows = dtw_chunk_rows(B, H, T);
  const int64_t n_chunks = (T + rows - 1) / rows;
  return align256((size_t)(B * H * T) * sizeof(float2)) + align256((size_t)(B * H * cpitch) * sizeof(float2)) +
         (size_t)(B * H * n_chunks * cpitch) * sizeof(float2);
}

void dtw_workspace_layout(void* ws, DtwArgs* a) {
  char* p = static_cast<char*>(ws);
  a->cpitch = (a->A + 3) & ~3;
  a->rc_rows = dtw_chunk_rows(a->B, a->H, a->T);
  const int64_t bh = (int64_t)a->B * a->H;
  a->rs = reinterpret_cast<float2*>(p);
  p += align256((size_t)(bh * a->T) * sizeof(float2));
  a->cs = reinterpret_cast<float2*>(p);
  p += align256((size_t)(bh * a->cpitch) * sizeof(float2));
  a->part = reinterpret_cast<float2*>(p);
}

hipError_t launch_dtw_prep(DtwArgs a, hipStream_t stream) {
  const int64_t n_rows = (int64_t)a.B * a.H * a.T;
  if (n_rows == 0 || a.C == 0) return hipSuccess;
  a.vec = (reinterpret_cast<uintptr_t>(a.w) & 15) == 0 && a.ws[0] % 4 == 0 && a.ws[1] % 4 == 0 &&
          a.ws[2] % 4 == 0;
  // Columns the filter reads: [0, min(A, C + pad)).
  const int need = a.C + a.pad < a.A ? a.C + a.pad : a.A;
  if (a.vec && a.A % 4 == 0 && a.A <= 2048) {
    a.rc_rows = dtw_chunk_rows(a.B, a.H, a.T, kRcSlotsRowcol);  // no more chunks than the workspace's
    const int64_t slab = (int64_t)a.H * a.T * a.A * 4;
    const int64_t keep = kMallKeepBytes / slab;
    a.nt_b = keep >= a.B ? 0 : (int)(a.B - keep);
    const dim3 grid((a.T + a.rc_rows - 1) / a.rc_rows, a.H, a.B);
    if (a.A <= 512) hipLaunchKernelGGL(dtw_rowcol_kernel<2>, grid, dim3(256), 0, stream, a);
    else if (a.A <= 1024) hipLaunchKernelGGL(dtw_rowcol_kernel<4>, grid, dim3(256), 0, stream, a);
    else if (a.A <= 1536) hipLaunchKernelGGL(dtw_rowcol_kernel<6>, grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(dtw_rowcol_kernel<8>, grid, dim3(256), 0, stream, a);
    hipLaunchKernelGGL(dtw_col_merge_kernel, dim3((need + 255) / 256, a.H, a.B), dim3(256), 0, stream, a, need);
  } else {
    const dim3 rgrid((unsigned)((n_rows + 3) / 4));
    if (a.vec) hipLaunchKernelGGL(dtw_row_stats_kernel<true>, rgrid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(dtw_row_stats_kernel<false>, rgrid, dim3(256), 0, stream, a);
    hipLaunchKernelGGL(dtw_col_stats_kernel, dim3((need + kColBlock - 1) / kColBlock, a.H, a.B), dim3(512), 0,
                       stream, a);
  }
  if (a.pad == 3 && a.A >= 4 * 64 && a.H <= kBandMaxHeads) {  // the reference's width 7
    const int n_seg = (a.C + kSegOut - 1) / kSegOut;
    const int64_t waves = (int64_t)a.B * ((a.T + kSegRows - 1) / kSegRows) * n_seg;
    hipLaunchKernelGGL(dtw_seg_kernel, dim3((unsigned)((waves + kSegWaves - 1) / kSegWaves)), dim3(kSegWaves * 64), 0,
                       stream, a, n_seg);
    return hipGetLastError();
  }
  if (a.vec && a.A % 4 == 0 && a.A <= 4 * kBandMaxA4 && a.H <= kBandMaxHeads) {
    const dim3 grid((a.T + kBandRows - 1) / kBandRows, a.B);
    if (a.pad == 3) {  // A < 256: one float4 column per thread
      hipLaunchKernelGGL((dtw_band_kernel<3, 128>), grid, dim3(128), 0, stream, a);
      return hipGetLastError();
    }
    switch (a.pad) {
#define WDRZ_BAND(P) \
  case P:            \
    hipLaunchKernelGGL((dtw_band_kernel<P, 512>), grid, dim3(512), 0, stream, a); \
    break;
      WDRZ_BAND(0) WDRZ_BAND(1) WDRZ_BAND(2) WDRZ_BAND(4) WDRZ_BAND(5) WDRZ_BAND(6) WDRZ_BAND(7)
#undef WDRZ_BAND
      default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
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

// Rows per chunk of the fused statistics pass: the two-pass chunking rounded up to whole 16-row
// blocks (never more chunks than the workspace holds).
static int dtw_qk_chunk_rows(int64_t B, int64_t H, int64_t T) {
  const int r = dtw_chunk_rows(B, H, T);
  return (r + 15) / 16 * 16;
}

hipError_t launch_dtw_qk_prep(int dtype, DtwArgs a, const DtwQkArgs& q, hipStream_t stream) {
  if ((int64_t)a.B * a.H * a.T == 0 || a.C == 0) return hipSuccess;
  if (a.A > kQkTilesPerWave * kQkWaves * 16) return hipErrorInvalidValue;
  a.rc_rows = dtw_qk_chunk_rows(a.B, a.H, a.T);
  const dim3 g1((unsigned)((a.T + a.rc_rows - 1) / a.rc_rows * a.H * a.B));
  if (dtype == 2) hipLaunchKernelGGL(dtw_qk_rowcol_kernel<Bf16>, g1, dim3(512), 0, stream, a, q);
  else hipLaunchKernelGGL(dtw_qk_rowcol_kernel<F16>, g1, dim3(512), 0, stream, a, q);
  const int need = a.C + a.pad < a.A ? a.C + a.pad : a.A;
  hipLaunchKernelGGL(dtw_col_merge_kernel, dim3((need + 255) / 256, a.H, a.B), dim3(256), 0, stream, a, need);
  const int64_t n2 = (int64_t)((a.C + kQsSeg - 1) / kQsSeg) * ((a.T + kQsRows - 1) / kQsRows) * a.B;
  const dim3 g2((unsigned)n2);
  switch (a.pad) {
#define WDRZ_QB(P)                                                                                   \
  case P:                                                                                            \
    if (dtype == 2) hipLaunchKernelGGL((dtw_qk_band_kernel<Bf16, P>), g2, dim3(256), 0, stream, a, q); \
    else hipLaunchKernelGGL((dtw_qk_band_kernel<F16, P>), g2, dim3(256), 0, stream, a, q);             \
    break;
    WDRZ_QB(0) WDRZ_QB(1) WDRZ_QB(2) WDRZ_QB(3) WDRZ_QB(4) WDRZ_QB(5) WDRZ_QB(6) WDRZ_QB(7)
#undef WDRZ_QB
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_median_filter(const MedianArgs& a, hipStream_t stream) {
  if (a.rows == 0 || a.N == 0) return hipSuccess;
  if (a.pad < 0 || a.pad > kDtwMaxPad) return hipErrorInvalidValue;
  MedianArgs v = a;
  v.vec = (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 &&
          a.xs % 4 == 0 && a.ys % 4 == 0;
  // one workgroup per row when it fits 2048 columns (64-lane steps), else 2048-column pieces
  int threads = (int)(((a.N + 3) / 4 + 63) / 64 * 64);
  threads = threads > kMfMaxThreads ? kMfMaxThreads : threads;
  const int64_t cols = 4 * threads;
  const int64_t n = (a.N + cols - 1) / cols * a.rows;
  if (n > 0x7fffffff) return hipErrorInvalidValue;
  switch (a.pad) {
#define WDRZ_MF(P) \
  case P:          \
    hipLaunchKernelGGL(median_filter_kernel<P>, dim3((unsigned)n), dim3(threads), 0, stream, v); \
    break;
    WDRZ_MF(0) WDRZ_MF(1) WDRZ_MF(2) WDRZ_MF(3) WDRZ_MF(4) WDRZ_MF(5) WDRZ_MF(6) WDRZ_MF(7)
#undef WDRZ_MF
  }
  return hipGetLastError();
}

}  // namespace wdrz
