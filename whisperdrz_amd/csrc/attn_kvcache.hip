// attn_kvcache.hip — split-KV attention for the decoder's cached paths (gfx950).
//
// Replaces flash_attn_with_kvcache / _sdpa_attn_with_kvcache (reference
// src/whisperdrz/model.py:20-95) for:
//   * cached self-attention with fused in-place append of k_new / v_new (model.py:49-63):
//     query t of batch row b sees keys j <= cache_seqlens[b] + t (bottom-right causal);
//   * cross-attention over the full cache (model.py:64-67), non-causal.
//
// The decode work is a GEMV per (b, h): every key row is touched once, so the kernel is HBM
// bound and uses no MFMA. A head row of K or V is 64 elements = one 16-byte load per lane
// across LPK lanes (8 lanes in 16-bit types, 16 in fp32). Lane groups of LPK lanes each own
// a strided subset of the keys, keep kUnroll keys in flight per batch and run an online
// softmax in the log2 domain; in 16-bit types q.k and P.V run on v_dot2 (P.V over key pairs).
//
// Launch shape: one 4-wavefront workgroup per (batch row, query block of up to 8, head, key
// split); its wavefront partials merge through LDS. Rows split their keys only when there are
// too few rows to fill the chip; a row with several splits has each split publish an (m, l, o)
// partial to the caller's workspace, and the split that arrives last (a per-row atomic
// counter) merges them, writes the output and resets the counter, all in the same launch.
//
// Append: keys at positions >= cache_seqlens[b] are read straight from k_new / v_new, never
// from the cache, so the in-place write (done by the split whose key range holds the row)
// cannot race with any read in the same launch.
//
// Which kernel serves a call (launch_typed): 16-bit calls of 2-8 query rows run on
// kv_mq_kernel (MFMA over the rows, below), 9-39 rows in its 16-row blocks when those alone fill
// the chip, and 40 or more rows (a prompt's self or cross attention) on kv_prefill_kernel in
// attn_dense.hip (256-query MFMA blocks); single rows, the remaining multi-row shapes and fp32
// caches run on kv_attn_kernel.
#include "kv_dup.h"
#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {

namespace {

constexpr int kMaxSQ = 8;  // query rows per workgroup
constexpr int kWavesPerWg = 4;   // wavefronts per workgroup
constexpr int kUnroll = 4;       // keys per lane group per batch (even: P V runs on key pairs)
constexpr int kMinSplitKeys = 128;
constexpr int kMaxMergeSplits = 32;  // upper bound on splits per row (host plan guarantees it)
constexpr float kTau = 8.0f;  // lazy-rescale threshold (log2 units)

// v_dot2 on packed 16-bit pairs with fp32 accumulation.
template <typename T> struct Dot2;
template <> struct Dot2<Bf16> {
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  static constexpr uint32_t kOnes = 0x3f803f80u;  // (1.0, 1.0)
  static __device__ __forceinline__ float run(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
};
template <> struct Dot2<F16> {
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static constexpr uint32_t kOnes = 0x3c003c00u;  // (1.0, 1.0)
  static __device__ __forceinline__ float run(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
};

// A quiet NaN built from its bit pattern (this file is compiled with -fno-honor-nans, under
// which a NaN literal would be undefined); it marks output rows with invalid metadata.
__device__ __forceinline__ float quiet_nan() { return __uint_as_float(0x7fc00000u); }

// In-place append (fused cache write) of query block [t0, t0 + nq) of batch row b, head h:
// thread i moves 16-byte piece i of the block's new K and V rows. The load is issued at kernel
// start, the store (by the split whose key range holds the row's position) after the key loop,
// so the load latency stays off the critical path.
struct AppendPiece {
  u32x4 v;
  bool on;
  int t, which, rr;  // query row in the block, K (0) or V (1), 16-byte piece in the head row
};
template <typename T>
__device__ __forceinline__ AppendPiece kv_append_load(const KvArgs& a, int b, int t0, int nq, int h) {
  constexpr int LPK = kHeadDim * ElemBytes<T>::value / 16;  // 16-byte pieces per head row
  AppendPiece p;
  const int idx = threadIdx.x;
  p.on = idx < nq * 2 * LPK;
  p.t = idx / (2 * LPK);
  p.which = (idx / LPK) & 1;
  p.rr = idx % LPK;
  p.v = u32x4{0, 0, 0, 0};
  if (p.on)
    p.v = load16((p.which ? a.vn + b * a.vns[0] + (int64_t)(t0 + p.t) * a.vns[1] + h * a.vns[2]
                          : a.kn + b * a.kns[0] + (int64_t)(t0 + p.t) * a.kns[1] + h * a.kns[2]) +
                 p.rr * 16);
  return p;
}
// `own`: this row stores its region (it is the last row appending there, kv_dup.h).
__device__ __forceinline__ void kv_append_store(const KvArgs& a, const AppendPiece& p, int t0, int h, int split,
                                                int slot, int cs, bool own) {
  const int lo = split * a.split_len, hi = lo + a.split_len;
  const int pos = cs + t0 + p.t;
  if (own && p.on && pos >= lo && pos < hi)
    store16((p.which ? a.vc + slot * a.vcs[0] + (int64_t)pos * a.vcs[1] + h * a.vcs[2]
                     : a.kc + slot * a.kcs[0] + (int64_t)pos * a.kcs[1] + h * a.kcs[2]) +
                p.rr * 16,
            p.v);
}

// Combines the per-wavefront partials (o[64], m, l per query, in LDS) of one workgroup and
// writes the output rows, or, when the row's keys are split over several workgroups,
// publishes this split's partial and lets the last split to arrive merge them all.
template <typename T, int SQ, int kWaves>
__device__ __forceinline__ void kv_finish(const KvArgs& a, int b, int t0, int nq, int sq_stride, int h, int split,
                                          int n_split_b, bool bad, float (&sm_acc)[kWaves][SQ][kHeadDim],
                                          float (&sm_m)[kWaves][SQ], float (&sm_l)[kWaves][SQ]) {
  constexpr int kThreads = kWaves * 64;
  constexpr int EB = ElemBytes<T>::value;
  constexpr int kPart = kHeadDim + 2;  // floats per partial: o[64], m, l
  __shared__ int sm_last;
  const int tid = threadIdx.x;
  auto store_out = [&](int t, int d, float val) {
    char* op = a.o + b * a.os[0] + (t0 + t) * a.os[1] + h * a.os[2];
    if constexpr (EB == 4)
      reinterpret_cast<float*>(op)[d] = val;
    else if constexpr (__is_same(T, Bf16))
      reinterpret_cast<__bf16*>(op)[d] = (__bf16)val;
    else
      reinterpret_cast<_Float16*>(op)[d] = (_Float16)val;
  };
  // This workgroup's (o, m, l) for query t, dim d, from the per-wavefront LDS partials.
  auto wg_partial = [&](int t, int d, float& O, float& M, float& L) {
    M = kNegBig;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][t]);
    L = 0.f;
    O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(sm_m[w][t] - M);
      L = __builtin_fmaf(sm_l[w][t], f, L);
      O = __builtin_fmaf(sm_acc[w][t][d], f, O);
    }
  };

  if (n_split_b == 1) {
    for (int idx = tid; idx < nq * kHeadDim; idx += kThreads) {
      const int t = idx / kHeadDim, d = idx % kHeadDim;
      float O, M, L;
      wg_partial(t, d, O, M, L);
      store_out(t, d, bad ? quiet_nan() : O / L);
    }
    return;
  }

  // ---- several splits: publish this split's partial; the last split to arrive merges ----
  // Partials are laid out with the workspace's row stride sq_stride (= the launch's query block,
  // which the host sized the workspace for; it can be smaller than SQ).
  const int64_t unit = ((int64_t)b * a.n_qblocks + t0 / sq_stride) * a.H + h;
  float* part = a.ws_part + (unit * a.n_splits) * (sq_stride * kPart);
  for (int idx = tid; idx < nq * kHeadDim; idx += kThreads) {
    const int t = idx / kHeadDim, d = idx % kHeadDim;
    float O, M, L;
    wg_partial(t, d, O, M, L);
    float* pp = part + (split * sq_stride + t) * kPart;
    __hip_atomic_store(pp + d, O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d == 0) {
      __hip_atomic_store(pp + kHeadDim, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(pp + kHeadDim + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // Ordering without cache maintenance: the partial was written with agent-scope atomic
  // stores, which complete at the device coherence point; waiting for them (vmcnt 0) before
  // the counter update makes it visible to whichever split reads the count last. (A C++
  // release fence here would write back the whole L2 of this XCD from every split.)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(a.ws_count + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm_last = prev == n_split_b - 1;
  }
  __syncthreads();
  if (!sm_last) return;
  // The merging workgroup reads the partials with agent-scope atomic loads (coherent, issued
  // only after the counter told it every partial had landed): first every (m, l) pair in
  // parallel into LDS, then one o value per (split, query, dim).
  __shared__ float sm_pm[kMaxMergeSplits * SQ], sm_pl[kMaxMergeSplits * SQ];
  for (int idx = tid; idx < n_split_b * nq; idx += kThreads) {
    const int sp = idx / nq, t = idx % nq;
    float* pp = part + (sp * sq_stride + t) * kPart;
    sm_pm[sp * SQ + t] = __hip_atomic_load(pp + kHeadDim, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm_pl[sp * SQ + t] = __hip_atomic_load(pp + kHeadDim + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    pp[kHeadDim] = 0.f;  // consumed: leave the workspace all-zero (see below)
    pp[kHeadDim + 1] = 0.f;
  }
  __syncthreads();
  for (int idx = tid; idx < nq * kHeadDim; idx += kThreads) {
    const int t = idx / kHeadDim, d = idx % kHeadDim;
    float mm = kNegBig;
    for (int sp = 0; sp < n_split_b; ++sp) mm = fmaxf(mm, sm_pm[sp * SQ + t]);
    float L = 0.f, O = 0.f;
    for (int sp = 0; sp < n_split_b; ++sp) {
      const float f = fast_exp2(sm_pm[sp * SQ + t] - mm);
      L = __builtin_fmaf(sm_pl[sp * SQ + t], f, L);
      float* po = part + (sp * sq_stride + t) * kPart + d;
      O = __builtin_fmaf(__hip_atomic_load(po, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), f, O);
      *po = 0.f;
    }
    store_out(t, d, O / L);
  }
  // Leave the counter at zero too. Every call returns the whole workspace to all-zero, so the
  // counters of any later call, whatever its shape and therefore its layout, start at zero.
  if (tid == 0) __hip_atomic_store(a.ws_count + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A row whose keys another row's append region overlaps other than exactly (kv_dup.h): the
// generic path computes its queries' partials into wavefront 0's LDS slots (the others empty),
// appends the positions this row wins, and hands over to the usual merge.
template <typename T, int SQ, int kWaves>
__device__ __forceinline__ void kv_general_row(const KvArgs& a, const AppendPiece& app, int b, int h, int slot, int cs,
                                               int t0, int nq, int sq_stride, int split, int n_split_b, int k_begin,
                                               int k_end, float (&sm_acc)[kWaves][SQ][kHeadDim], float (&sm_m)[kWaves][SQ],
                                               float (&sm_l)[kWaves][SQ]) {
  __shared__ float sm_q[kWaves][kHeadDim];
  kv_generic_rows<T, kWaves>(a, b, h, slot, cs, t0, nq, k_begin, k_end, true, sm_q,
                             [&](int t, int d, float o, float m, float l) {
                               sm_acc[0][t][d] = o;
                               if (d == 0) {
                                 sm_m[0][t] = m;
                                 sm_l[0][t] = l;
                               }
                             });
  for (int idx = threadIdx.x; idx < (kWaves - 1) * SQ * kHeadDim; idx += kWaves * 64) {
    const int w = 1 + idx / (SQ * kHeadDim), t = (idx / kHeadDim) % SQ, d = idx % kHeadDim;
    sm_acc[w][t][d] = 0.f;
    if (d == 0) {
      sm_m[w][t] = kNegBig;
      sm_l[w][t] = 0.f;
    }
  }
  int cw = 0;
  const bool own = app.on && kv_dup_winner(a, slot, cs + t0 + app.t, cw) == b;
  kv_append_store(a, app, t0, h, split, slot, cs, own);
  __syncthreads();
  kv_finish<T, SQ, kWaves>(a, b, t0, nq, sq_stride, h, split, n_split_b, false, sm_acc, sm_m, sm_l);
}

template <typename T, int SQ, bool HAS_NEW>
__global__ __launch_bounds__(kWavesPerWg * 64) void kv_attn_kernel(KvArgs a) {
  constexpr int kThreads = kWavesPerWg * 64;
  constexpr int kWaves = kWavesPerWg;
  constexpr int EB = ElemBytes<T>::value;
  constexpr int EPL = 16 / EB;         // elements per lane per 16-byte load
  constexpr int LPK = kHeadDim / EPL;  // lanes per key row
  constexpr int G = kThreads / LPK;    // key groups per workgroup

  __shared__ float sm_acc[kWaves][SQ][kHeadDim];
  __shared__ float sm_m[kWaves][SQ];
  __shared__ float sm_l[kWaves][SQ];

  const int tid = threadIdx.x;
  const int g = tid / LPK;
  const int r = tid % LPK;
  const int wave = tid / 64;
  const int lane = tid % 64;

  // Heads fastest in the dispatch order: the workgroups running at once read one slot's heads,
  // which lie next to each other in the head-major cache (config 3: 17.4 -> 15.5 us against
  // batch rows fastest).
  const int h = (int)(blockIdx.x % (unsigned)a.H);
  const int bq = (int)(blockIdx.x / (unsigned)a.H);
  const int b = bq / a.n_qblocks;
  const int t0 = (bq % a.n_qblocks) * SQ;
  const int split = blockIdx.z;
  const int nq = min(SQ, a.sq - t0);

  const int slot = a.bidx ? a.bidx[b] : b;
  const int cs = HAS_NEW ? a.seqlens[b] : 0;
  // other rows appending to this slot (kv_dup.h): usually none
  const KvDup dup = HAS_NEW ? kv_dup_classify(a, b, slot, cs) : KvDup{b, false};
  // Loads that need no metadata are issued while it arrives: the queries and the rows to
  // append (stored after the key loop, when they have long arrived).
  u32x4 qraw[SQ];
#pragma unroll
  for (int t = 0; t < SQ; ++t) {
    const int tt = t0 + min(t, nq - 1);
    qraw[t] = load16(a.q + b * a.qs[0] + tt * a.qs[1] + h * a.qs[2] + r * 16);
  }
  static_assert(kMaxSQ * 2 * LPK <= kThreads, "one append piece per thread");
  const AppendPiece app = HAS_NEW ? kv_append_load<T>(a, b, t0, nq, h) : AppendPiece{};
  // Metadata the host cannot validate without reading device memory. A bad row produces NaN
  // output instead of touching memory outside the cache.
  const bool bad = slot < 0 || slot >= a.n_slots || cs < 0 || (HAS_NEW && cs + a.sq > a.Lk);

  // Keys this query block needs: [0, key_lim).
  const int key_lim = HAS_NEW ? cs + t0 + nq : a.Lk;
  // Splits that hold keys of this row; the others have nothing to do.
  const int n_split_b = bad ? 1 : max(1, (key_lim + a.split_len - 1) / a.split_len);
  if (split >= n_split_b) return;
  const int k_begin = split * a.split_len;
  const int k_end = bad ? k_begin : min(key_lim, k_begin + a.split_len);
  if (HAS_NEW && dup.general && !bad) {
    kv_general_row<T, SQ, kWaves>(a, app, b, h, slot, cs, t0, nq, SQ, split, n_split_b, k_begin, k_end, sm_acc,
                                  sm_m, sm_l);
    return;
  }

  // Queries. 16-bit types keep the raw packed pairs for v_dot2 (the scale is applied to the
  // reduced score); fp32 keeps floats pre-scaled into the log2 domain.
  float qf[SQ][EPL];
#pragma unroll
  for (int t = 0; t < SQ; ++t) {
    if constexpr (EB == 4) {
      Slice<T> sl;
      sl.from_raw(qraw[t]);
#pragma unroll
      for (int e = 0; e < EPL; ++e) qf[t][e] = sl.v[e] * a.c;
    }
  }

  // Per query: running max (log2 units), partial row sum and output slice of this lane group.
  float m[SQ], l[SQ], acc[SQ][EPL];
#pragma unroll
  for (int t = 0; t < SQ; ++t) {
    m[t] = kNegBig;
    l[t] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[t][e] = 0.f;
  }
  // Last key each query may see inside this split (inclusive).
  int lim[SQ];
#pragma unroll
  for (int t = 0; t < SQ; ++t) {
    lim[t] = k_end - 1;
    if (HAS_NEW) lim[t] = min(lim[t], cs + t0 + t);
  }

  const int safe_slot = bad ? 0 : slot;
  const char* kc_row = a.kc + safe_slot * a.kcs[0] + h * a.kcs[2] + r * 16;
  const char* vc_row = a.vc + safe_slot * a.vcs[0] + h * a.vcs[2] + r * 16;
  // the appended rows: those of the last row appending this same region (this row when alone)
  const char* kn_row = HAS_NEW ? a.kn + dup.src * a.kns[0] + h * a.kns[2] + r * 16 : nullptr;
  const char* vn_row = HAS_NEW ? a.vn + dup.src * a.vns[0] + h * a.vns[2] + r * 16 : nullptr;

  // Batches of kUnroll keys per lane group. Loads past the row's end re-read its last key.
  auto load_batch = [&](int base, u32x4 (&kr)[kUnroll], u32x4 (&vr)[kUnroll]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int kk = min(base + u * G, k_end - 1);
      const char* kp;
      const char* vp;
      if (HAS_NEW && kk >= cs) {
        kp = kn_row + (int64_t)(kk - cs) * a.kns[1];
        vp = vn_row + (int64_t)(kk - cs) * a.vns[1];
      } else {
        kp = kc_row + (int64_t)kk * a.kcs[1];
        vp = vc_row + (int64_t)kk * a.vcs[1];
      }
      kr[u] = load16_stream(kp);
      vr[u] = load16_stream(vp);
    }
  };
  auto compute_batch = [&](int base, const u32x4 (&kr)[kUnroll], const u32x4 (&vr)[kUnroll]) __attribute__((always_inline)) {
    // ---- scores (log2 units), masked to -inf outside each query's key range ----
    float sc[SQ][kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if constexpr (EB == 2) {
#pragma unroll
        for (int t = 0; t < SQ; ++t) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) d = Dot2<T>::run(qraw[t][i], kr[u][i], d);
          sc[t][u] = group_sum<LPK>(d) * a.c;
        }
      } else {
        Slice<T> ks;
        ks.from_raw(kr[u]);
#pragma unroll
        for (int t = 0; t < SQ; ++t) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < EPL; ++e) d = __builtin_fmaf(qf[t][e], ks.v[e], d);
          sc[t][u] = group_sum<LPK>(d);
        }
      }
#pragma unroll
      for (int t = 0; t < SQ; ++t)
        if (base + u * G > lim[t]) sc[t][u] = -INFINITY;
    }
    // ---- lazy max update: move the reference only when a score exceeds it by > kTau ----
    float mb[SQ];
    bool grow = false;
#pragma unroll
    for (int t = 0; t < SQ; ++t) {
      mb[t] = sc[t][0];
#pragma unroll
      for (int u = 1; u < kUnroll; ++u) mb[t] = fmaxf(mb[t], sc[t][u]);
      grow = grow || mb[t] > m[t] + kTau;
    }
    if (__any(grow)) {
#pragma unroll
      for (int t = 0; t < SQ; ++t) {
        const float mn = mb[t] > m[t] + kTau ? mb[t] : m[t];
        const float alpha = fast_exp2(m[t] - mn);
        m[t] = mn;
        l[t] *= alpha;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[t][e] *= alpha;
      }
    }
    // ---- P V ----
    if constexpr (EB == 2) {
      // Keys in pairs: v_perm gathers dim e of both keys into one dword, v_dot2 multiplies it
      // with the packed pair of probabilities.
#pragma unroll
      for (int u = 0; u < kUnroll; u += 2) {
        u32x4 vlo, vhi;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          vlo[i] = __builtin_amdgcn_perm(vr[u + 1][i], vr[u][i], 0x05040100u);
          vhi[i] = __builtin_amdgcn_perm(vr[u + 1][i], vr[u][i], 0x07060302u);
        }
#pragma unroll
        for (int t = 0; t < SQ; ++t) {
          const uint32_t pp = Dot2<T>::pack(fast_exp2(sc[t][u] - m[t]), fast_exp2(sc[t][u + 1] - m[t]));
          l[t] = Dot2<T>::run(pp, Dot2<T>::kOnes, l[t]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[t][2 * i] = Dot2<T>::run(pp, vlo[i], acc[t][2 * i]);
            acc[t][2 * i + 1] = Dot2<T>::run(pp, vhi[i], acc[t][2 * i + 1]);
          }
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        Slice<T> vs;
        vs.from_raw(vr[u]);
#pragma unroll
        for (int t = 0; t < SQ; ++t) {
          const float p = fast_exp2(sc[t][u] - m[t]);
          l[t] += p;
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[t][e] = __builtin_fmaf(p, vs.v[e], acc[t][e]);
        }
      }
    }
  };
  constexpr int kStride = G * kUnroll;
  if constexpr (SQ == 1) {
    // Decode rows: software-pipelined, the next batch's loads in flight while the current one
    // is computed (one workgroup streams a long row ~15% faster; +32 registers).
    u32x4 kA[kUnroll], vA[kUnroll], kB[kUnroll], vB[kUnroll];
    int base = k_begin + g;
    if (base < k_end) load_batch(base, kA, vA);
    for (; base < k_end; base += 2 * kStride) {
      const bool more = base + kStride < k_end;
      if (more) load_batch(base + kStride, kB, vB);
      compute_batch(base, kA, vA);
      if (!more) break;
      if (base + 2 * kStride < k_end) load_batch(base + 2 * kStride, kA, vA);
      compute_batch(base + kStride, kB, vB);
    }
  } else {
    for (int base = k_begin + g; base < k_end; base += kStride) {
      u32x4 kr[kUnroll], vr[kUnroll];
      load_batch(base, kr, vr);
      compute_batch(base, kr, vr);
    }
  }

  if (HAS_NEW && !bad) kv_append_store(a, app, t0, h, split, slot, cs, dup.src == b);

  // Merge lane groups inside the wavefront (groups differ in lane bits >= log2(LPK)).
#pragma unroll
  for (int off = LPK; off < 64; off *= 2) {
#pragma unroll
    for (int t = 0; t < SQ; ++t) {
      const float mo = __shfl_xor(m[t], off);
      const float lo = __shfl_xor(l[t], off);
      const float mn = fmaxf(m[t], mo);
      const float fa = fast_exp2(m[t] - mn), fb = fast_exp2(mo - mn);
      l[t] = l[t] * fa + lo * fb;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[t][e] = acc[t][e] * fa + __shfl_xor(acc[t][e], off) * fb;
      m[t] = mn;
    }
  }
  if (lane < LPK) {
#pragma unroll
    for (int t = 0; t < SQ; ++t) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) sm_acc[wave][t][r * EPL + e] = acc[t][e];
      if (r == 0) {
        sm_m[wave][t] = m[t];
        sm_l[wave][t] = l[t];
      }
    }
  }
  __syncthreads();

  kv_finish<T, SQ, kWaves>(a, b, t0, nq, SQ, h, split, n_split_b, bad, sm_acc, sm_m, sm_l);
}

// ============================================================================================
// Multi-query rows on the matrix core (16-bit types: 2 <= sq <= 8 in one block, the draft
// verify; longer prefills in blocks of 16 rows when those blocks fill the chip, see the C layer).
// With several queries per row the VALU form above spends most of its time on the
// per-query dot products, reductions and exps of every key; here a wavefront takes 32 keys
// per step and computes
//   S^T (32 keys x 16 query slots) = K . Q^T       with 4 v_mfma_f32_16x16x32,
//   O^T (64 dims x 16 query slots) += V^T . P^T    with 4 more,
// so the VALU only runs the softmax of 8 scores per lane. K rows feed the A operand straight
// from global memory (lane l: key l%16 of a 16-key block, dims 8*(l/16)..+7 of a 32-dim half);
// V rows go through a per-wavefront LDS tile and come back transposed by ds_read_b64_tr_b16.
// The P^T operand is the S^T accumulator itself: lane l holds query l%16 and keys
// 4*(l/16)..+3 of each 16-key block, i.e. keys {4g..4g+3, 16+4g..16+4g+3} for g = l/16, and the
// V^T operand is read in that same key order. Query slots past the block's rows are computed and
// discarded.
// The four wavefronts of a workgroup take interleaved 32-key chunks of the row (or split);
// their partials merge through LDS as in the VALU kernel.
// ============================================================================================
constexpr int kMqChunk = 32;                   // keys per wavefront step
constexpr int kMqPitch = kHeadDim + 8;         // V tile row pitch (elements)

template <typename T> struct Mfma16;
template <> struct Mfma16<Bf16> {
  typedef bf16x8 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma16<F16> {
  typedef f16x8 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group, lane i receives element
// i%4 of the 8-byte chunks read by lanes 4c + i/4 (c = 0..3). `p` must point into __shared__
// memory (its low 32 bits are the LDS byte address).
__device__ __forceinline__ u32x2 kv_read_tr16(const uint16_t* p) {
#if __HIP_DEVICE_COMPILE__
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uint32_t)(uintptr_t)p));
#else
  (void)p;
  return u32x2{0, 0};
#endif
}

// max of x over lanes l, l^16, l^32, l^48 (the four 16-lane groups), in every lane
__device__ __forceinline__ float group4_max(float x) {
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
}

// SQ: query rows per workgroup, 8 (one block of sq <= 8 rows) or 16 (blocks of 16 rows of a
// longer prefill; every MFMA query slot used).
template <typename T, bool HAS_NEW, int SQ>
// At most 128 VGPRs (four wavefronts per SIMD): measured 5% faster for config 5 than the
// unconstrained 148 (three per SIMD, the row's 1280 workgroups then need 1.7 rounds).
__global__ __launch_bounds__(kWavesPerWg * 64, 4) void kv_mq_kernel(KvArgs a) {
  typedef typename Mfma16<T>::op_t op_t;
  constexpr int kWaves = kWavesPerWg;
  static_assert(SQ <= 16, "16 query slots per MFMA tile");
  __shared__ float sm_acc[kWaves][SQ][kHeadDim];
  __shared__ float sm_m[kWaves][SQ];
  __shared__ float sm_l[kWaves][SQ];
  __shared__ __attribute__((aligned(16))) uint16_t sm_v[kWaves][kMqChunk * kMqPitch];

  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int qi = lane & 15;  // query slot of this lane
  const int gq = lane >> 4;  // 16-lane group

  const int h = (int)(blockIdx.x % (unsigned)a.H);  // heads fastest, as in kv_attn_kernel
  const int bq = (int)(blockIdx.x / (unsigned)a.H);
  const int b = bq / a.n_qblocks;
  const int t0 = (bq % a.n_qblocks) * SQ;  // first query row of this block
  const int split = blockIdx.z;
  const int nq = min(SQ, a.sq - t0);

  const int slot = a.bidx ? a.bidx[b] : b;
  const int cs = HAS_NEW ? a.seqlens[b] : 0;
  const KvDup dup = HAS_NEW ? kv_dup_classify(a, b, slot, cs) : KvDup{b, false};
  static_assert(SQ * 2 * (kHeadDim * 2 / 16) <= kWaves * 64, "one append piece per thread");
  const AppendPiece app = HAS_NEW ? kv_append_load<T>(a, b, t0, nq, h) : AppendPiece{};
  const bool bad = slot < 0 || slot >= a.n_slots || cs < 0 || (HAS_NEW && cs + a.sq > a.Lk);
  const int key_lim = HAS_NEW ? cs + t0 + nq : a.Lk;
  const int n_split_b = bad ? 1 : max(1, (key_lim + a.split_len - 1) / a.split_len);
  if (split >= n_split_b) return;
  const int k_begin = split * a.split_len;
  const int k_end = bad ? k_begin : min(key_lim, k_begin + a.split_len);
  if (HAS_NEW && dup.general && !bad) {
    kv_general_row<T, SQ, kWaves>(a, app, b, h, slot, cs, t0, nq, a.n_qblocks > 1 ? SQ : nq, split, n_split_b,
                                  k_begin, k_end, sm_acc, sm_m, sm_l);
    return;
  }
  // last key this lane's query may see (slots >= nq see none)
  int lim = k_end - 1;
  if (HAS_NEW) lim = min(lim, cs + t0 + qi);
  if (qi >= nq) lim = -1;

  // Q^T operand halves: query t0 + qi (clamped), dims 32*dh + 8*gq .. +7
  op_t qop[2];
  {
    const char* qrow = a.q + b * a.qs[0] + (t0 + min(qi, nq - 1)) * a.qs[1] + h * a.qs[2];
#pragma unroll
    for (int dh = 0; dh < 2; ++dh) qop[dh] = __builtin_bit_cast(op_t, load16(qrow + (32 * dh + 8 * gq) * 2));
  }

  const int safe_slot = bad ? 0 : slot;
  const char* kc_row = a.kc + safe_slot * a.kcs[0] + h * a.kcs[2];
  const char* vc_row = a.vc + safe_slot * a.vcs[0] + h * a.vcs[2];
  const char* kn_row = HAS_NEW ? a.kn + dup.src * a.kns[0] + h * a.kns[2] : nullptr;  // see kv_attn_kernel
  const char* vn_row = HAS_NEW ? a.vn + dup.src * a.vns[0] + h * a.vns[2] : nullptr;
  auto k_ptr = [&](int key) __attribute__((always_inline)) {
    return (HAS_NEW && key >= cs) ? kn_row + (int64_t)(key - cs) * a.kns[1] : kc_row + (int64_t)key * a.kcs[1];
  };
  auto v_ptr = [&](int key) __attribute__((always_inline)) {
    return (HAS_NEW && key >= cs) ? vn_row + (int64_t)(key - cs) * a.vns[1] : vc_row + (int64_t)key * a.vcs[1];
  };

  // Loads of one 32-key chunk: K operands (kop[kb][dh]: key kb*16 + l%16, 16 bytes at dims
  // 32*dh + 8*(l/16)) and this lane's four 16-byte pieces of the V tile (rows (l + 64*i)/8).
  op_t kop[2][2];
  u32x4 vld[4];
  auto load_chunk = [&](int key0) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const char* kp = k_ptr(min(key0 + kb * 16 + qi, k_end - 1));
#pragma unroll
      for (int dh = 0; dh < 2; ++dh) kop[kb][dh] = __builtin_bit_cast(op_t, load16_stream(kp + (32 * dh + 8 * gq) * 2));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int piece = lane + 64 * i;
      vld[i] = load16_stream(v_ptr(min(key0 + (piece >> 3), k_end - 1)) + (piece & 7) * 16);
    }
  };
  uint16_t* vt = sm_v[wave];
  // transposing-read base for this lane: key row 4*gq + (j>>2) (+16 for the second read), dims
  // 4*(j&3) of each 16-dim block, j = lane index in its 16-lane group
  const uint16_t* vt_lane = vt + (4 * gq + (qi >> 2)) * kMqPitch + 4 * (qi & 3);

  float m = kNegBig, l = 0.f;
  f32x4 o[4];  // O^T blocks: dims 16*db + 4*gq + i, query qi
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int stride = kWaves * kMqChunk;
  int key0 = k_begin + wave * kMqChunk;
  if (key0 < k_end) load_chunk(key0);
  for (; key0 < k_end; key0 += stride) {
    // V tile of this chunk into LDS ([key][dim], padded rows)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int piece = lane + 64 * i;
      *reinterpret_cast<u32x4*>(&vt[(piece >> 3) * kMqPitch + (piece & 7) * 8]) = vld[i];
    }
    // ---- S^T = K Q^T for the two 16-key blocks ----
    f32x4 sblk[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sblk[kb] = Mfma16<T>::run(kop[kb][0], qop[0], f32x4{0.f, 0.f, 0.f, 0.f});
      sblk[kb] = Mfma16<T>::run(kop[kb][1], qop[1], sblk[kb]);
    }
    // next chunk's loads (registers are free once the MFMAs above are issued)
    if (key0 + stride < k_end) load_chunk(key0 + stride);
    // ---- V^T operands (same key order as P^T) ----
    op_t vop[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const u32x2 lo = kv_read_tr16(vt_lane + 16 * db);
      const u32x2 hi = kv_read_tr16(vt_lane + 16 * kMqPitch + 16 * db);
      vop[db] = __builtin_bit_cast(op_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
    }
    // ---- softmax of the lane's 8 scores (log2 units), masked past each query's limit ----
    float sc[8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = key0 + kb * 16 + 4 * gq + i;
        sc[kb * 4 + i] = key <= lim ? sblk[kb][i] * a.c : -INFINITY;
      }
    float mb = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
    mb = group4_max(mb);
    if (__any(mb > m + kTau)) {
      asm volatile("" ::: "memory");  // keep this rare path a branch
      const float mn = mb > m + kTau ? mb : m;
      const float alpha = fast_exp2(m - mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    }
    uint32_t pw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pw[j] = Dot2<T>::pack(fast_exp2(sc[2 * j] - m), fast_exp2(sc[2 * j + 1] - m));
      l = Dot2<T>::run(pw[j], Dot2<T>::kOnes, l);
    }
    const op_t pop = __builtin_bit_cast(op_t, u32x4{pw[0], pw[1], pw[2], pw[3]});
    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = Mfma16<T>::run(vop[db], pop, o[db]);
  }

  if (HAS_NEW && !bad) kv_append_store(a, app, t0, h, split, slot, cs, dup.src == b);

  // row sums: the four lane groups hold different keys of the same query
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (qi < nq) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) sm_acc[wave][qi][16 * db + 4 * gq + i] = o[db][i];
    if (gq == 0) {
      sm_m[wave][qi] = m;
      sm_l[wave][qi] = l;
    }
  }
  __syncthreads();
  kv_finish<T, SQ, kWaves>(a, b, t0, nq, a.n_qblocks > 1 ? SQ : nq, h, split, n_split_b, bad, sm_acc, sm_m, sm_l);
}

template <typename T>
hipError_t launch_typed(const KvArgs& a, hipStream_t stream) {
  const int64_t n_units = (int64_t)a.B * a.n_qblocks * a.H;
  if (n_units > 0x7fffffff) return hipErrorInvalidValue;
  dim3 grid((unsigned)n_units, 1, a.n_splits);
  const bool has_new = a.kn != nullptr;
  const int sq_blk = a.n_qblocks > 1 ? kMaxSQ : a.sq;
  if constexpr (ElemBytes<T>::value == 2) {
    // many queries (a prompt's self and cross attention): 256-query MFMA blocks (attn_dense.hip),
    // each key row read ~sq/256 times instead of once per 16-query block
    if (a.sq >= kPrefillMinSq) return launch_kv_prefill(__is_same(T, Bf16) ? 2 : 1, a, stream);
    if (a.mq_rows == 16) {  // prefill in 16-row blocks on the matrix cores
      if (has_new)
        hipLaunchKernelGGL((kv_mq_kernel<T, true, 16>), grid, dim3(kWavesPerWg * 64), 0, stream, a);
      else
        hipLaunchKernelGGL((kv_mq_kernel<T, false, 16>), grid, dim3(kWavesPerWg * 64), 0, stream, a);
      return hipGetLastError();
    }
    if (a.n_qblocks == 1 && sq_blk >= 2) {
      if (has_new)
        hipLaunchKernelGGL((kv_mq_kernel<T, true, kMaxSQ>), grid, dim3(kWavesPerWg * 64), 0, stream, a);
      else
        hipLaunchKernelGGL((kv_mq_kernel<T, false, kMaxSQ>), grid, dim3(kWavesPerWg * 64), 0, stream, a);
      return hipGetLastError();
    }
  }
#define WDRZ_KV_CASE(SQV)                                                                       \
  case SQV:                                                                                     \
    if (has_new)                                                                                \
      hipLaunchKernelGGL((kv_attn_kernel<T, SQV, true>), grid, dim3(kWavesPerWg * 64), 0, stream, a); \
    else                                                                                         \
      hipLaunchKernelGGL((kv_attn_kernel<T, SQV, false>), grid, dim3(kWavesPerWg * 64), 0, stream, a); \
    break;
  switch (sq_blk) {
    WDRZ_KV_CASE(1)
    WDRZ_KV_CASE(2)
    WDRZ_KV_CASE(3)
    WDRZ_KV_CASE(4)
    WDRZ_KV_CASE(5)
    WDRZ_KV_CASE(6)
    WDRZ_KV_CASE(7)
    WDRZ_KV_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef WDRZ_KV_CASE
  return hipGetLastError();
}

}  // namespace

void kv_split_plan(int64_t units, int64_t Lk, int* n_splits, int* split_len) {
  // One workgroup per row walks all its keys when there are enough rows to fill the chip
  // (splitting costs a partial round trip per split and, measured, never pays off then).
  // Fewer rows split their keys so that >= 1024 workgroups (four per CU) are in flight.
  const int64_t max_splits = (Lk + kMinSplitKeys - 1) / kMinSplitKeys;
  int64_t want = (1024 + units - 1) / (units > 0 ? units : 1);
  if (want < 1) want = 1;
  if (want > max_splits) want = max_splits;
  if (want > kMaxMergeSplits) want = kMaxMergeSplits;
  int64_t len = (Lk + want - 1) / want;
  len = (len + 63) / 64 * 64;
  *split_len = (int)len;
  *n_splits = (int)((Lk + len - 1) / len);
  if (*n_splits < 1) *n_splits = 1;
}

size_t kv_workspace_bytes(int64_t units, int64_t sq_blk, int n_splits) {
  if (n_splits <= 1) return 0;
  const size_t counters = ((size_t)units * sizeof(int) + 255) / 256 * 256;
  return counters + (size_t)units * n_splits * sq_blk * (kHeadDim + 2) * sizeof(float);
}

void kv_workspace_layout(void* ws, int64_t units, KvArgs* a) {
  const size_t counters = ((size_t)units * sizeof(int) + 255) / 256 * 256;
  a->ws_count = static_cast<int*>(ws);
  a->ws_part = reinterpret_cast<float*>(static_cast<char*>(ws) + counters);
}

hipError_t launch_kv_attn(int dtype, const KvArgs& a, hipStream_t stream) {
  switch (dtype) {
    case 0:
      return launch_typed<F32>(a, stream);
    case 1:
      return launch_typed<F16>(a, stream);
    case 2:
      return launch_typed<Bf16>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace wdrz
