// kv_fill.hip — writing projected K/V rows into the slot caches.
//
// Replaces FlashKVCache.prefill / set_cross_attention (src/whisperdrz/model.py:150-183):
//   k_cache[slot_indices[b], start + t] = k[b, t],  v_cache[...] = v[b, t]
// which torch runs as an index_put into the caches (a scatter over a permuted view when the
// cache is stored head-major, as KVSlotPool stores it). The cross fill after each encoder pass
// (prefill_flash, model.py:851-862) moves 2 x B x 1500 x 1280 elements per layer this way.
//
// One 256-lane workgroup per (32 rows of t, head, b): lane (r, c) moves the 16-byte chunk c of
// row t0 + r of K and of V. The source rows of one head are 128-byte pieces of the [B, T, H, D]
// projection output; the destination rows of one (slot, head) are consecutive 128-byte rows of a
// head-major cache, so a workgroup writes one contiguous 4 KB run per tensor. Both sides are
// touched once: nontemporal loads and stores. Slot ids outside [0, n_slots) are skipped (device
// data the host cannot check without a synchronisation).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {
namespace {

constexpr int kFillRows = 32;

__global__ __launch_bounds__(256) void kv_fill_kernel(KvFillArgs a) {
  const int tb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int r = threadIdx.x >> 3, c = threadIdx.x & 7;  // row in the block, 16-byte chunk
  const int t = tb * kFillRows + r;
  if (t >= a.T) return;
  const int64_t slot = a.slots ? a.slots[b] : b;
  if (slot < 0 || slot >= a.n_slots) return;
  const int64_t src = (int64_t)b * a.ss[0] + (int64_t)t * a.ss[1] + (int64_t)h * a.ss[2] + c * 8;
  const int64_t dst = slot * a.cs[0] + (int64_t)(a.start + t) * a.cs[1] + (int64_t)h * a.cs[2] + c * 8;
  const uint16_t* ks = static_cast<const uint16_t*>(a.k_src);
  const uint16_t* vs = static_cast<const uint16_t*>(a.v_src);
  const u32x4 kw = load16_stream(ks + src);
  const u32x4 vw = load16_stream(vs + src);
  __builtin_nontemporal_store(kw, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.k_cache) + dst));
  __builtin_nontemporal_store(vw, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.v_cache) + dst));
}

}  // namespace

hipError_t launch_kv_fill(const KvFillArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.T == 0 || a.H == 0) return hipSuccess;
  const dim3 grid((unsigned)((a.T + kFillRows - 1) / kFillRows), (unsigned)a.H, (unsigned)a.B);
  hipLaunchKernelGGL(kv_fill_kernel, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace wdrz
