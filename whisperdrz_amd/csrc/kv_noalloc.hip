// kv_noalloc.hip — the cached-attention entry point for callers that cannot allocate.
//
// wdrz_attn_kvcache_noalloc is wdrz_attn_kvcache with its split-KV workspace taken from a
// file-scope device array instead of a caller buffer: code under graph capture without an
// allocator, tight serving loops, harnesses that forbid hipMalloc. It runs the same kernels.
//
// The array holds the per-row arrival counters and the (m, l, o) partials of the split path.
// Its size bounds every workspace the split plan can ask for: rows are split only while
// B * ceil(sq/8) * H < 1024, so units * splits < 2048, and the partials take at most
// 2048 * 8 queries * 66 floats * 4 B = 4.33 MB. The kernels leave it all-zero after every call,
// so it is cleared once per device, when the device's address is first taken.
//
// Each GPU holds its own copy of the array (at its own address) until the process ends, and
// every call on a GPU uses that GPU's copy: calls that overlap on one GPU (two streams, two
// threads) race on it. Serialise them, or use wdrz_attn_kvcache with separate workspaces.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/wdrz_attn.h"
#include "wdrz_launch.h"

namespace {

constexpr size_t kScratchBytes = WDRZ_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ void clear_kernel(uint4* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = uint4{0u, 0u, 0u, 0u};
}

std::mutex g_mu;
void* g_ptr[kMaxDevices];  // device address of `scratch`, per device (nullptr: not set up)

// The device address of this device's scratch array, taken (and the array cleared on
// `stream`) on the first call for the device. Returns a WDRZ_* code.
int scratch_for_current_device(hipStream_t stream, void** out, const char** why) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *why = "no current HIP device";
    return WDRZ_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *why = "hipGetSymbolAddress failed for the scratch array";
      return WDRZ_ELAUNCH;
    }
    // A kernel, not a memset: the first call may be under graph capture.
    hipLaunchKernelGGL(clear_kernel, dim3(256), dim3(256), 0, stream, static_cast<uint4*>(p),
                       kScratchBytes / sizeof(uint4));
    if (hipGetLastError() != hipSuccess) {
      *why = "clearing the scratch array failed";
      return WDRZ_ELAUNCH;
    }
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return WDRZ_OK;
}

}  // namespace

extern "C" {

int wdrz_attn_kvcache_noalloc(int dtype, const void* q, void* k_cache, void* v_cache, const void* k_new,
                              const void* v_new, const int32_t* cache_seqlens, const int32_t* cache_batch_idx,
                              void* o, int64_t B, int64_t sq, int64_t H, int64_t D, int64_t n_slots, int64_t Lmax,
                              const int64_t* q_strides, const int64_t* kc_strides, const int64_t* vc_strides,
                              const int64_t* kn_strides, const int64_t* vn_strides, const int64_t* o_strides,
                              float softmax_scale, int causal, void* stream) {
  const size_t need = wdrz_attn_kvcache_workspace_size(B, sq, H, D, Lmax);
  if (need > kScratchBytes)
    return wdrz::set_last_error(WDRZ_EUNSUPPORTED, "split workspace of %zu bytes exceeds the %zu-byte static scratch",
                                need, kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const char* why = "";
    const int rc = scratch_for_current_device(reinterpret_cast<hipStream_t>(stream), &ws, &why);
    if (rc != WDRZ_OK) return wdrz::set_last_error(rc, "%s", why);
  }
  return wdrz_attn_kvcache(dtype, q, k_cache, v_cache, k_new, v_new, cache_seqlens, cache_batch_idx, o, B, sq, H, D,
                           n_slots, Lmax, q_strides, kc_strides, vc_strides, kn_strides, vn_strides, o_strides,
                           softmax_scale, causal, ws, need > 0 ? kScratchBytes : 0, stream);
}

}  // extern "C"
