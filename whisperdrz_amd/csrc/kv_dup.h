// kv_dup.h — batch rows of one cached-attention call that name the same cache slot.
//
// The reference fallback appends batch row by batch row and only then gathers the keys
// (src/whisperdrz/model.py:49-57): with repeated cache_batch_idx entries position p of slot s ends
// up holding the new row of the LAST batch row i with cache_batch_idx[i] == s and
// cache_seqlens[i] <= p < cache_seqlens[i] + sq (or its old contents when no row covers p), and
// every row attends over that final cache. The kernels follow the same rule without ever reading a
// position that another workgroup writes in the same launch:
//   * rows whose slot no other row names, or only rows with the same append region (the padded
//     rows of a bucketed decode graph repeat a stale slot id with that slot's own length,
//     transcriber.py:76-78, 165-167): the usual path, except that the region's keys and values are
//     read from the last of those rows (`src`), and only that row stores them;
//   * any other overlap (another row's region starts before this row's last key): a generic
//     per-workgroup path (kv_generic_rows) that resolves every key position to its winner.
#pragma once

#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {

// A row appends to `slot` when it names it and its region [cs, cs + sq) lies inside the cache
// (rows with invalid metadata produce NaN and append nothing).
__device__ __forceinline__ bool kv_dup_appends(const KvArgs& a, int slot_i, int cs_i, int slot) {
  return slot_i == slot && slot >= 0 && slot < a.n_slots && cs_i >= 0 && cs_i + a.sq <= a.Lk;
}

struct KvDup {
  int src;       // the last batch row appending exactly this row's region (this row when alone)
  bool general;  // another row's region overlaps this row's keys otherwise: generic path
};

// Wave-level: every lane must be active; the result is the same in every lane and in every
// wavefront of the workgroup.
__device__ __forceinline__ KvDup kv_dup_classify(const KvArgs& a, int b, int slot, int cs) {
  KvDup d{b, false};
  if (a.kn == nullptr || a.bidx == nullptr) return d;
  const int lane = threadIdx.x & 63;
  bool gen = false;
  auto chunk = [&](int base, bool in, int si, int ci) __attribute__((always_inline)) {
    const bool app = in && kv_dup_appends(a, si, ci, slot);
    gen = gen || (app && ci != cs && ci < cs + a.sq);
    const uint64_t m = __ballot(app && ci == cs);
    if (m) d.src = max(d.src, base + 63 - __clzll((long long)m));
  };
  // the first 64 rows with unconditional (clamped) loads, so they issue with the row's own
  // metadata; larger batches loop
  const int i0 = min(lane, a.B - 1);
  chunk(0, lane < a.B, a.bidx[i0], a.seqlens[i0]);
  for (int base = 64; base < a.B; base += 64) {
    const int i = min(base + lane, a.B - 1);
    chunk(base, base + lane < a.B, a.bidx[i], a.seqlens[i]);
  }
  d.general = __ballot(gen) != 0ull;
  return d;
}

// The batch row whose new row holds position p of `slot` once every row has appended (the last
// row covering p), with its cache_seqlens in cs_w; -1 when no row covers p (the cache's own
// contents). Per lane, uniform loop over the batch (scalar loads); generic path only.
__device__ __forceinline__ int kv_dup_winner(const KvArgs& a, int slot, int p, int& cs_w) {
  int w = -1;
  for (int i = 0; i < a.B; ++i) {
    const int ci = a.seqlens[i];
    if (kv_dup_appends(a, a.bidx[i], ci, slot) && p >= ci && p < ci + a.sq) {
      w = i;
      cs_w = ci;
    }
  }
  return w;
}

template <int W>
__device__ __forceinline__ float kv_wave_max(float x) {
#pragma unroll
  for (int off = W / 2; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}
template <int W>
__device__ __forceinline__ float kv_wave_sum(float x) {
#pragma unroll
  for (int off = W / 2; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

template <typename T>
__device__ __forceinline__ float kv_elem(const char* row, int d) {
  if constexpr (ElemBytes<T>::value == 4)
    return reinterpret_cast<const float*>(row)[d];
  else if constexpr (__is_same(T, Bf16))
    return (float)reinterpret_cast<const __bf16*>(row)[d];
  else
    return (float)reinterpret_cast<const _Float16*>(row)[d];
}

// Generic cached attention of batch row b, head h, query rows t0 + [0, nq), over keys
// [k_begin, k_end) (self: query t also stops at cs + t0 + t), every key position resolved to the
// row that wins it. One wavefront per query (rows dealt round-robin over the workgroup's
// wavefronts); in each batch of 64 keys a lane computes one key's score, then the lanes take the
// 64 head dimensions for P.V. emit(t, d, o, m, l) receives, in lane d, the unnormalised output
// and the running max (log2 units) and sum, as the fast paths keep them for their merge. q_lds: 64
// floats of LDS per wavefront. Slow (latency-bound): used only for the overlapping appends above.
template <typename T, int kWaves, typename Emit>
__device__ __forceinline__ void kv_generic_rows(const KvArgs& a, int b, int h, int slot, int cs, int t0, int nq,
                                                int k_begin, int k_end, bool self_attn, float (*q_lds)[kHeadDim],
                                                Emit emit) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const char* kc_row = a.kc + (int64_t)slot * a.kcs[0] + (int64_t)h * a.kcs[2];
  const char* vc_row = a.vc + (int64_t)slot * a.vcs[0] + (int64_t)h * a.vcs[2];
  for (int t = wave; t < nq; t += kWaves) {
    q_lds[wave][lane] = kv_elem<T>(a.q + (int64_t)b * a.qs[0] + (int64_t)(t0 + t) * a.qs[1] + (int64_t)h * a.qs[2], lane) * a.c;
    __builtin_amdgcn_wave_barrier();
    const int kend = self_attn ? min(k_end, cs + t0 + t + 1) : k_end;
    float m = kNegBig, l = 0.f, acc = 0.f;  // kNegBig: "no key yet", as the fast paths keep it
    for (int kb = k_begin; kb < kend; kb += 64) {
      const int j = kb + lane;
      const bool valid = j < kend;
      const char* kp = kc_row + (int64_t)j * a.kcs[1];
      const char* vp = vc_row + (int64_t)j * a.vcs[1];
      if (self_attn && valid) {
        int cw = 0;
        const int w = kv_dup_winner(a, slot, j, cw);
        if (w >= 0) {
          kp = a.kn + (int64_t)w * a.kns[0] + (int64_t)(j - cw) * a.kns[1] + (int64_t)h * a.kns[2];
          vp = a.vn + (int64_t)w * a.vns[0] + (int64_t)(j - cw) * a.vns[1] + (int64_t)h * a.vns[2];
        }
      }
      float s = -INFINITY;
      if (valid) {
        float dot = 0.f;
        for (int d = 0; d < kHeadDim; ++d) dot = __builtin_fmaf(q_lds[wave][d], kv_elem<T>(kp, d), dot);
        s = dot;
      }
      const float mn = fmaxf(m, kv_wave_max<64>(s));
      const float alpha = fast_exp2(m - mn);
      const float p = valid ? fast_exp2(s - mn) : 0.f;
      l = l * alpha + kv_wave_sum<64>(p);
      acc *= alpha;
      m = mn;
      const uint64_t vlo = (uint64_t)(uintptr_t)vp;
      const int n = min(64, kend - kb);
      for (int jj = 0; jj < n; ++jj) {
        const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), jj));
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)vlo, jj);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(vlo >> 32), jj);
        const char* vrow = reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
        acc = __builtin_fmaf(pj, kv_elem<T>(vrow, lane), acc);
      }
    }
    emit(t, lane, acc, m, l);
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace wdrz
