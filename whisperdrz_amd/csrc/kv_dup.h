// kv_dup.h — batch rows of one cached-attention call that name the same cache slot.
//
// The reference fallback appends batch row by batch row and only then gathers the keys
// (src/whisperdrz/model.py:49-57): with repeated cache_batch_idx entries (the padded rows of a
// bucketed decode graph carry stale slot ids, transcriber.py:76-78, 165-167) position p of slot s
// ends up holding the new row of the LAST batch row i with cache_batch_idx[i] == s and
// cache_seqlens[i] <= p < cache_seqlens[i] + sq, or its old contents when no row covers p, and every
// row attends over that final cache. The kernels follow the same rule without ever reading a
// position that another workgroup writes in the same launch: a covered position is read from its
// winner's k_new / v_new, and only the winner stores it.
//
// kv_dup_scan runs once per wavefront at kernel start (all 64 lanes active). When no other row
// shares the slot the window is empty and the kernels take their usual path: key p < cs from the
// cache, p >= cs from this row's own k_new.
#pragma once

#include "wdrz_launch.h"

#include <limits.h>

namespace wdrz {

struct KvDup {
  int lo, hi;      // positions [lo, hi) are appended by OTHER rows sharing the slot (lo >= hi: none)
  uint64_t rows;   // B <= 64: the rows (self included) that append to this slot with valid metadata
  int cs_lane;     // B <= 64: cache_seqlens of batch row `lane`
};

// A row appends to `slot` when it names it and its region [cs, cs + sq) lies inside the cache
// (rows with invalid metadata produce NaN and append nothing).
__device__ __forceinline__ bool kv_dup_appends(const KvArgs& a, int slot_i, int cs_i, int slot) {
  return slot_i == slot && cs_i >= 0 && cs_i + a.sq <= a.Lk;
}

// Wave-level: every lane must be active; the result is the same in every lane. The window is
// gathered with scalar reads of the lanes that hold matching rows (no cross-lane shuffles on the
// common path, where no other row names the slot).
__device__ __forceinline__ KvDup kv_dup_scan(const KvArgs& a, int b, int slot) {
  KvDup d{INT_MAX, INT_MIN, 0ull, 0};
  if (a.kn == nullptr || a.bidx == nullptr) return d;
  const int lane = threadIdx.x & 63;
  for (int base = 0; base < a.B; base += 64) {
    const int i = base + lane;
    int ci = 0;
    bool mine = false;
    if (i < a.B) {
      ci = a.seqlens[i];
      mine = kv_dup_appends(a, a.bidx[i], ci, slot);
    }
    const uint64_t m = __ballot(mine);
    if (base == 0) {
      d.rows = m;
      d.cs_lane = ci;
    }
    uint64_t others = (b >= base && b < base + 64) ? m & ~(1ull << (b - base)) : m;
    while (others) {
      const int j = 63 - __clzll((long long)others);
      others &= ~(1ull << j);
      const int cj = __builtin_amdgcn_readlane(ci, j);
      d.lo = min(d.lo, cj);
      d.hi = max(d.hi, cj + a.sq);
    }
  }
  return d;
}

// The batch row whose new row holds position p of `slot` once every row has appended (the last
// row covering p), with its cache_seqlens in cs_w; -1 when no row covers p (the cache's own
// contents). Per lane; may run under divergence (it reads lanes with v_readlane only).
__device__ __forceinline__ int kv_dup_winner(const KvArgs& a, const KvDup& d, int slot, int p, int& cs_w) {
  if (a.B <= 64) {
    uint64_t m = d.rows;
    while (m) {
      const int i = 63 - __clzll((long long)m);
      m &= ~(1ull << i);
      const int ci = __builtin_amdgcn_readlane(d.cs_lane, i);
      if (p >= ci && p < ci + a.sq) {
        cs_w = ci;
        return i;
      }
    }
    return -1;
  }
  for (int i = a.B - 1; i >= 0; --i) {
    const int ci = a.seqlens[i];
    if (kv_dup_appends(a, a.bidx[i], ci, slot) && p >= ci && p < ci + a.sq) {
      cs_w = ci;
      return i;
    }
  }
  return -1;
}

__device__ __forceinline__ bool kv_dup_in_window(const KvDup& d, int p) { return p >= d.lo && p < d.hi; }

}  // namespace wdrz
