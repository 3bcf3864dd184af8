// wdrz_capi.cpp — the extern "C" boundary of libwdrz_attn.so (declared in include/wdrz_attn.h).
//
// Host-side only: validates every argument that can be checked without reading device memory,
// converts element strides to byte strides, and forwards to the kernel launchers. Nothing here
// allocates, frees, synchronises or reads device memory, so the entry points may be called
// during hipGraph stream capture.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/wdrz_attn.h"
#include "wdrz_launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int elem_bytes(int dtype) {
  switch (dtype) {
    case WDRZ_F32:
      return 4;
    case WDRZ_F16:
    case WDRZ_BF16:
      return 2;
    default:
      return 0;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks a 4-stride tensor description (element strides): last stride 1, others 16-B aligned.
int check_strides(const char* name, const int64_t* s, int eb) {
  if (!s) return fail(WDRZ_EINVAL, "%s: strides pointer is NULL", name);
  if (s[3] != 1) return fail(WDRZ_EINVAL, "%s: head_dim stride must be 1 (got %lld)", name, (long long)s[3]);
  for (int i = 0; i < 3; ++i) {
    if (((s[i] * eb) & 15) != 0)
      return fail(WDRZ_EINVAL, "%s: stride[%d]=%lld elements is not 16-byte aligned", name, i, (long long)s[i]);
  }
  return WDRZ_OK;
}

int check_ptr(const char* name, const void* p) {
  if (!p) return fail(WDRZ_EINVAL, "%s is NULL", name);
  if (!aligned16(p)) return fail(WDRZ_EINVAL, "%s is not 16-byte aligned", name);
  return WDRZ_OK;
}

// Validates what wdrz_dtw_prep and wdrz_dtw_attention_prep share and fills the DtwArgs (no
// scores pointer). Returns WDRZ_OK, an error code, or -1 for "nothing to do".
int dtw_common_args(const int32_t* actual_lens, const int32_t* audio_caps, float* out, const int64_t* out_strides,
                    int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int medfilt_width, void* workspace,
                    size_t workspace_bytes, wdrz::DtwArgs* a) {
  if (B < 0 || H <= 0 || T < 0 || A <= 0 || C < 0)
    return fail(WDRZ_EINVAL, "bad sizes B=%lld H=%lld T=%lld A=%lld C=%lld", (long long)B, (long long)H,
                (long long)T, (long long)A, (long long)C);
  if (C > A) return fail(WDRZ_EINVAL, "C=%lld exceeds A=%lld", (long long)C, (long long)A);
  if (T > wdrz::kDtwMaxRows)
    return fail(WDRZ_EUNSUPPORTED, "T=%lld text rows exceed the supported %d", (long long)T, wdrz::kDtwMaxRows);
  if (B > 65535 || H > 65535 || A > (1 << 24) || B * H * T > (int64_t(1) << 31))
    return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (medfilt_width < 1 || (medfilt_width > 1 && medfilt_width % 2 == 0))
    return fail(WDRZ_EINVAL, "medfilt_width=%d must be 1 or odd", medfilt_width);
  if (medfilt_width / 2 > wdrz::kDtwMaxPad)
    return fail(WDRZ_EUNSUPPORTED, "medfilt_width=%d exceeds the supported %d", medfilt_width,
                2 * wdrz::kDtwMaxPad + 1);
  if (!out) return fail(WDRZ_EINVAL, "out is NULL");
  if (!actual_lens || !audio_caps) return fail(WDRZ_EINVAL, "actual_lens / audio_caps is NULL");
  if (!out_strides) return fail(WDRZ_EINVAL, "strides pointer is NULL");
  if (out_strides[2] != 1) return fail(WDRZ_EINVAL, "out: last stride must be 1");
  if (B == 0 || T == 0 || C == 0) return -1;
  const size_t need = wdrz::dtw_workspace_bytes(B, H, T, A);
  if (!workspace || workspace_bytes < need)
    return fail(WDRZ_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace ? workspace_bytes : 0);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(WDRZ_EINVAL, "workspace is not 256-byte aligned");
  a->lens = actual_lens;
  a->caps = audio_caps;
  a->out = out;
  a->B = (int)B;
  a->H = (int)H;
  a->T = (int)T;
  a->A = (int)A;
  a->C = (int)C;
  const int pad = medfilt_width / 2;
  a->pad = (medfilt_width > 1 && A > pad) ? pad : 0;  // dtw_align.py:68-69: too short -> unfiltered
  a->os[0] = out_strides[0];
  a->os[1] = out_strides[1];
  wdrz::dtw_workspace_layout(workspace, a);
  return WDRZ_OK;
}

// q/k head pointer arrays and strides for the alignment heads (shared by the two QK entry points).
int dtw_qk_heads(int dtype, const void* const* q_heads, const int64_t* q_strides, const void* const* k_heads,
                 const int64_t* k_strides, int64_t H, int64_t D, wdrz::DtwQkArgs* a) {
  if (dtype != WDRZ_BF16 && dtype != WDRZ_F16)
    return fail(dtype == WDRZ_F32 ? WDRZ_EUNSUPPORTED : WDRZ_EINVAL,
                "dtype %d: only WDRZ_BF16 / WDRZ_F16 projections are supported", dtype);
  if (D != 64) return fail(WDRZ_EUNSUPPORTED, "head_dim %lld is not supported (only 64)", (long long)D);
  if (H <= 0) return fail(WDRZ_EINVAL, "bad head count %lld", (long long)H);
  if (H > wdrz::kDtwMaxHeads)
    return fail(WDRZ_EUNSUPPORTED, "%lld heads exceed the supported %d", (long long)H, wdrz::kDtwMaxHeads);
  if (!q_heads || !k_heads) return fail(WDRZ_EINVAL, "q_heads / k_heads is NULL");
  if (!q_strides || !k_strides) return fail(WDRZ_EINVAL, "strides pointer is NULL");
  if (q_strides[2] != 1 || k_strides[2] != 1) return fail(WDRZ_EINVAL, "q/k: head_dim stride must be 1");
  for (int i = 0; i < 2; ++i)
    if (((q_strides[i] * 2) & 15) || ((k_strides[i] * 2) & 15))
      return fail(WDRZ_EINVAL, "q/k: stride[%d] is not 16-byte aligned", i);
  for (int64_t h = 0; h < H; ++h) {
    int rc;
    if ((rc = check_ptr("q_heads[h]", q_heads[h])) || (rc = check_ptr("k_heads[h]", k_heads[h]))) return rc;
    a->q[h] = q_heads[h];
    a->k[h] = k_heads[h];
  }
  a->qs[0] = q_strides[0];
  a->qs[1] = q_strides[1];
  a->ks[0] = k_strides[0];
  a->ks[1] = k_strides[1];
  return WDRZ_OK;
}
#ifdef WDRZ_DEBUG_CHECKS
// Copies the slot ids and pre-append lengths of a cached-attention call to the host
// (synchronously) and checks every row: slot in [0, n_slots), length >= 0, and with an append
// length + sq <= Lmax. Rows that name the same slot are valid: the kernels apply their appends in
// batch order, as the reference fallback does (model.py:51-54).
int debug_check_kv_metadata(const int32_t* seqlens, const int32_t* bidx, bool has_new, int64_t B, int64_t sq,
                            int64_t n_slots, int64_t Lmax) {
  std::vector<int32_t> hs(B, 0), hb(B);
  for (int64_t i = 0; i < B; ++i) hb[i] = (int32_t)i;
  if (bidx && hipMemcpy(hb.data(), bidx, B * sizeof(int32_t), hipMemcpyDeviceToHost) != hipSuccess)
    return fail(WDRZ_ELAUNCH, "debug check: reading cache_batch_idx failed");
  if (has_new && hipMemcpy(hs.data(), seqlens, B * sizeof(int32_t), hipMemcpyDeviceToHost) != hipSuccess)
    return fail(WDRZ_ELAUNCH, "debug check: reading cache_seqlens failed");
  for (int64_t i = 0; i < B; ++i) {
    if (hb[i] < 0 || hb[i] >= n_slots)
      return fail(WDRZ_EINVAL, "debug check: row %lld names slot %d outside [0, %lld)", (long long)i, hb[i],
                  (long long)n_slots);
    if (has_new && (hs[i] < 0 || hs[i] + sq > Lmax))
      return fail(WDRZ_EINVAL, "debug check: row %lld appends [%d, %lld) outside the cache [0, %lld)", (long long)i,
                  hs[i], (long long)(hs[i] + sq), (long long)Lmax);
  }
  return WDRZ_OK;
}
#endif

}  // namespace

namespace wdrz {
int set_last_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}
}  // namespace wdrz

extern "C" {

const char* wdrz_last_error(void) { return g_last_error.c_str(); }

int wdrz_abi_version(void) { return 1; }

#ifndef WDRZ_BUILD_ID
#define WDRZ_BUILD_ID "unknown"
#endif
const char* wdrz_build_id(void) { return WDRZ_BUILD_ID; }

int wdrz_attn_fwd(int dtype, const void* q, const void* k, const void* v, void* o, int64_t B, int64_t H,
                  int64_t Lq, int64_t Lk, int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                  const int64_t* v_strides, const int64_t* o_strides, float scale, int causal, void* stream) {
  g_last_error.clear();
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(WDRZ_EINVAL, "dtype %d is not one of WDRZ_F32/F16/BF16", dtype);
  if (D != 64) return fail(WDRZ_EUNSUPPORTED, "head_dim %lld is not supported (only 64)", (long long)D);
  if (B < 0 || H <= 0 || Lq < 0 || Lk <= 0)
    return fail(WDRZ_EINVAL, "bad sizes B=%lld H=%lld Lq=%lld Lk=%lld", (long long)B, (long long)H,
                (long long)Lq, (long long)Lk);
  if (B > 65535 || H > 65535 || Lq > (1 << 24) || Lk > (1 << 24))
    return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (!(scale > 0.f) || scale != scale) return fail(WDRZ_EINVAL, "scale must be a positive finite number");
  int rc;
  if ((rc = check_ptr("q", q)) || (rc = check_ptr("k", k)) || (rc = check_ptr("v", v)) || (rc = check_ptr("o", o)))
    return rc;
  if ((rc = check_strides("q", q_strides, eb)) || (rc = check_strides("k", k_strides, eb)) ||
      (rc = check_strides("v", v_strides, eb)) || (rc = check_strides("o", o_strides, eb)))
    return rc;
  if (B == 0 || Lq == 0) return WDRZ_OK;
  const float c = scale * 1.4426950408889634f;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t err;
  {
    wdrz::DenseArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.B = (int)B;
    a.H = (int)H;
    a.Lq = (int)Lq;
    a.Lk = (int)Lk;
    a.causal = causal ? 1 : 0;
    const int64_t* S[4] = {q_strides, k_strides, v_strides, o_strides};
    int64_t* Dst[4] = {a.qs, a.ks, a.vs, a.os};
    for (int i = 0; i < 4; ++i)
      for (int j = 0; j < 3; ++j) Dst[i][j] = S[i][j];
    a.c = c;
    // fp32 on the fp32 matrix cores, 16-bit types on the bf16 / fp16 ones
    err = dtype == WDRZ_F32 ? wdrz::launch_dense_f32(a, st) : wdrz::launch_dense_mfma(dtype, a, st);
  }
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

size_t wdrz_attn_kvcache_workspace_size(int64_t B, int64_t sq, int64_t H, int64_t D, int64_t Lmax) {
  (void)D;
  if (B <= 0 || sq <= 0 || H <= 0 || Lmax <= 0) return 0;
  // kPrefillMinSq or more query rows never split their keys (16-bit types run them on the
  // 256-query prefill kernel, fp32 on one workgroup per 8-row block): no workspace
  if (sq >= wdrz::kPrefillMinSq) return 0;
  const int64_t n_qblocks = (sq + 7) / 8;
  const int64_t units = B * n_qblocks * H;
  int n_splits, split_len;
  wdrz::kv_split_plan(units, Lmax, &n_splits, &split_len);
  return wdrz::kv_workspace_bytes(units, sq < 8 ? sq : 8, n_splits);
}

int wdrz_attn_kvcache(int dtype, const void* q, void* k_cache, void* v_cache, const void* k_new, const void* v_new,
                      const int32_t* cache_seqlens, const int32_t* cache_batch_idx, void* o, int64_t B, int64_t sq,
                      int64_t H, int64_t D, int64_t n_slots, int64_t Lmax, const int64_t* q_strides,
                      const int64_t* kc_strides, const int64_t* vc_strides, const int64_t* kn_strides,
                      const int64_t* vn_strides, const int64_t* o_strides, float softmax_scale, int causal,
                      void* workspace, size_t workspace_bytes, void* stream) {
  (void)causal;
  g_last_error.clear();
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(WDRZ_EINVAL, "dtype %d is not one of WDRZ_F32/F16/BF16", dtype);
  if (D != 64) return fail(WDRZ_EUNSUPPORTED, "head_dim %lld is not supported (only 64)", (long long)D);
  if (B < 0 || sq <= 0 || H <= 0 || n_slots <= 0 || Lmax <= 0)
    return fail(WDRZ_EINVAL, "bad sizes B=%lld sq=%lld H=%lld n_slots=%lld Lmax=%lld", (long long)B,
                (long long)sq, (long long)H, (long long)n_slots, (long long)Lmax);
  if (B > (1 << 20) || H > 65535 || sq > 4096 || Lmax > (1 << 24) || n_slots > (1 << 24))
    return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (!(softmax_scale > 0.f) || softmax_scale != softmax_scale)
    return fail(WDRZ_EINVAL, "softmax_scale must be a positive finite number");
  const bool has_new = k_new != nullptr || v_new != nullptr;
  if (has_new && (!k_new || !v_new)) return fail(WDRZ_EINVAL, "k and v must be given together");
  if (has_new && !cache_seqlens) return fail(WDRZ_EINVAL, "cache_seqlens is required when k/v are given");
  if (has_new && sq > Lmax) return fail(WDRZ_EINVAL, "sq=%lld exceeds cache length %lld", (long long)sq, (long long)Lmax);
  int rc;
  if ((rc = check_ptr("q", q)) || (rc = check_ptr("k_cache", k_cache)) || (rc = check_ptr("v_cache", v_cache)) ||
      (rc = check_ptr("out", o)))
    return rc;
  if ((rc = check_strides("q", q_strides, eb)) || (rc = check_strides("k_cache", kc_strides, eb)) ||
      (rc = check_strides("v_cache", vc_strides, eb)) || (rc = check_strides("out", o_strides, eb)))
    return rc;
  if (has_new) {
    if ((rc = check_ptr("k", k_new)) || (rc = check_ptr("v", v_new))) return rc;
    if ((rc = check_strides("k", kn_strides, eb)) || (rc = check_strides("v", vn_strides, eb))) return rc;
  }
  if (B == 0) return WDRZ_OK;
#ifdef WDRZ_DEBUG_CHECKS
  // Debug build: check the device metadata on the host before launching (the release kernels
  // turn a bad row into NaN output without touching memory outside the caches).
  if ((rc = debug_check_kv_metadata(cache_seqlens, cache_batch_idx, has_new, B, sq, n_slots, Lmax))) return rc;
#endif

  wdrz::KvArgs a{};
  a.q = static_cast<const char*>(q);
  a.kc = static_cast<char*>(k_cache);
  a.vc = static_cast<char*>(v_cache);
  a.kn = has_new ? static_cast<const char*>(k_new) : nullptr;
  a.vn = has_new ? static_cast<const char*>(v_new) : nullptr;
  a.seqlens = has_new ? cache_seqlens : nullptr;
  a.bidx = cache_batch_idx;
  a.o = static_cast<char*>(o);
  a.B = (int)B;
  a.sq = (int)sq;
  a.H = (int)H;
  a.Lk = (int)Lmax;
  a.n_slots = (int)n_slots;
  // Prefill (sq > 8) in 16-bit types runs on the multi-query MFMA kernel in 16-row blocks when
  // those blocks fill the chip on their own (so the launch never splits its keys and needs no
  // workspace); otherwise in blocks of 8 rows, as the workspace size query assumes.
  const bool mq16 = eb == 2 && sq > 8 && B * ((sq + 15) / 16) * H >= 1024;
  a.n_qblocks = (int)(mq16 ? (sq + 15) / 16 : (sq + 7) / 8);
  a.mq_rows = mq16 ? 16 : 0;
  const int64_t* S[4] = {q_strides, kc_strides, vc_strides, o_strides};
  int64_t* Dst[4] = {a.qs, a.kcs, a.vcs, a.os};
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 3; ++j) Dst[i][j] = S[i][j] * eb;
  if (has_new)
    for (int j = 0; j < 3; ++j) {
      a.kns[j] = kn_strides[j] * eb;
      a.vns[j] = vn_strides[j] * eb;
    }
  a.c = softmax_scale * 1.4426950408889634f;
  const int64_t units = B * a.n_qblocks * H;
  if (units > 0x7fffffff) return fail(WDRZ_EUNSUPPORTED, "B * ceil(sq / rows per block) * H exceeds 2^31 - 1");
  if (sq >= wdrz::kPrefillMinSq) {  // never split (see wdrz_attn_kvcache_workspace_size)
    a.n_splits = 1;
    a.split_len = (int)Lmax;
  } else {
    wdrz::kv_split_plan(units, Lmax, &a.n_splits, &a.split_len);
  }
  const size_t need = wdrz::kv_workspace_bytes(units, sq < 8 ? sq : 8, a.n_splits);
  if (need > 0) {
    if (!workspace || workspace_bytes < need)
      return fail(WDRZ_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace ? workspace_bytes : 0);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return fail(WDRZ_EINVAL, "workspace is not 256-byte aligned");
    wdrz::kv_workspace_layout(workspace, units, &a);
  }
  hipError_t err = wdrz::launch_kv_attn(dtype, a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

int wdrz_dtw_qk(int dtype, const void* const* q_heads, const int64_t* q_strides, const void* const* k_heads,
                const int64_t* k_strides, float* out, const int64_t* out_strides, int64_t B, int64_t H, int64_t T,
                int64_t A, int64_t D, float scale, void* stream) {
  g_last_error.clear();
  if (B < 0 || T < 0 || A < 0)
    return fail(WDRZ_EINVAL, "bad sizes B=%lld T=%lld A=%lld", (long long)B, (long long)T, (long long)A);
  wdrz::DtwQkArgs a{};
  int rc = dtw_qk_heads(dtype, q_heads, q_strides, k_heads, k_strides, H, D, &a);
  if (rc != WDRZ_OK) return rc;
  if (B * H > 65535 || T > (1 << 24) || A > (1 << 24)) return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (!(scale > 0.f) || scale != scale) return fail(WDRZ_EINVAL, "scale must be a positive finite number");
  if (!out_strides) return fail(WDRZ_EINVAL, "strides pointer is NULL");
  if (!out) return fail(WDRZ_EINVAL, "out is NULL");
  if (out_strides[3] != 1) return fail(WDRZ_EINVAL, "out: last stride must be 1");
  if (B == 0 || T == 0 || A == 0) return WDRZ_OK;
  a.out = out;
  a.B = (int)B;
  a.H = (int)H;
  a.T = (int)T;
  a.A = (int)A;
  for (int i = 0; i < 3; ++i) a.os[i] = out_strides[i];
  a.scale2 = scale * scale;
  hipError_t err = wdrz::launch_dtw_qk(dtype, a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

int wdrz_add_layernorm(int dtype, void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                       const void* weight, const void* bias, void* y, int64_t y_stride, int64_t rows, int64_t n,
                       float eps, void* stream) {
  g_last_error.clear();
  if (dtype != WDRZ_BF16 && dtype != WDRZ_F16)
    return fail(dtype == WDRZ_F32 ? WDRZ_EUNSUPPORTED : WDRZ_EINVAL, "dtype %d: only WDRZ_BF16 / WDRZ_F16", dtype);
  if (rows < 0 || n <= 0 || n % 8 != 0)
    return fail(WDRZ_EINVAL, "bad sizes rows=%lld n=%lld (n must be a positive multiple of 8)", (long long)rows,
                (long long)n);
  if (n > 4096) return fail(WDRZ_EUNSUPPORTED, "n=%lld exceeds the supported 4096", (long long)n);
  if (!(eps >= 0.f)) return fail(WDRZ_EINVAL, "eps must be >= 0");
  int rc;
  if ((rc = check_ptr("x", x)) || (rc = check_ptr("weight", weight)) || (rc = check_ptr("bias", bias)) ||
      (rc = check_ptr("y", y)))
    return rc;
  if (delta && (rc = check_ptr("delta", delta))) return rc;
  if ((x_stride * 2) % 16 || (y_stride * 2) % 16 || (delta && (delta_stride * 2) % 16))
    return fail(WDRZ_EINVAL, "row strides must be 16-byte aligned");
  if (rows > 1 && (x_stride < n || y_stride < n || (delta && delta_stride < n)))
    return fail(WDRZ_EINVAL, "row strides shorter than the rows");
  if (rows == 0) return WDRZ_OK;
  wdrz::AddLnArgs a{};
  a.x = x;
  a.delta = delta;
  a.weight = weight;
  a.bias = bias;
  a.y = y;
  a.rows = rows;
  a.n = (int)n;
  a.x_stride = x_stride;
  a.d_stride = delta_stride;
  a.y_stride = y_stride;
  a.eps = eps;
  hipError_t err = wdrz::launch_add_layernorm(dtype, a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

int wdrz_masked_argmax(int dtype, const void* logits, int64_t logits_stride, const uint8_t* blocked,
                       int64_t blocked_stride, const uint8_t* penalty, int64_t penalty_stride, int64_t* out,
                       int64_t rows, int64_t V, void* stream) {
  g_last_error.clear();
  if (!elem_bytes(dtype)) return fail(WDRZ_EINVAL, "dtype %d is not one of WDRZ_F32/F16/BF16", dtype);
  if (rows < 0 || V <= 0) return fail(WDRZ_EINVAL, "bad sizes rows=%lld V=%lld", (long long)rows, (long long)V);
  if (rows > (1 << 24) || V > (1 << 30)) return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (!logits || !out) return fail(WDRZ_EINVAL, "logits / out is NULL");
  if (rows == 0) return WDRZ_OK;
  wdrz::ArgmaxArgs a{};
  a.logits = logits;
  a.l_stride = logits_stride;
  a.blocked = blocked;
  a.m_stride = blocked_stride;
  a.penalty = penalty;
  a.p_stride = penalty_stride;
  a.out = out;
  a.rows = (int)rows;
  a.V = (int)V;
  hipError_t err = wdrz::launch_masked_argmax(dtype, a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

int wdrz_linear(int dtype, const void* x, int64_t x_stride, const void* w, int64_t w_stride, const void* bias,
                void* y, int64_t y_stride, int64_t M, int64_t N, int64_t K, int activation, void* stream) {
  g_last_error.clear();
  if (dtype != WDRZ_BF16 && dtype != WDRZ_F16)
    return fail(dtype == WDRZ_F32 ? WDRZ_EUNSUPPORTED : WDRZ_EINVAL, "dtype %d: only WDRZ_BF16 / WDRZ_F16", dtype);
  if (activation != 0 && activation != 1) return fail(WDRZ_EINVAL, "activation %d is not 0 (none) or 1 (GELU)", activation);
  if (M < 0 || N <= 0 || K <= 0) return fail(WDRZ_EINVAL, "bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  if (K % 128 != 0 || N % 8 != 0)
    return fail(WDRZ_EUNSUPPORTED, "K=%lld must be a multiple of 128 and N=%lld of 8", (long long)K, (long long)N);
  // ceil(M / 64) row blocks go in grid.y, which holds at most 65535
  if (M > 65535 * 64 || N > (1 << 24) || K > (1 << 20)) return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (M == 0) return WDRZ_OK;  // nothing to read or write (an empty tensor's pointer may be NULL)
  int rc;
  if ((rc = check_ptr("x", x)) || (rc = check_ptr("w", w)) || (rc = check_ptr("y", y))) return rc;
  if (bias && (reinterpret_cast<uintptr_t>(bias) & 1)) return fail(WDRZ_EINVAL, "bias is not 2-byte aligned");
  if (x_stride < K || w_stride < K || y_stride < N) return fail(WDRZ_EINVAL, "row strides shorter than the rows");
  if ((x_stride * 2) % 16 || (w_stride * 2) % 16 || (y_stride * 2) % 16)
    return fail(WDRZ_EINVAL, "row strides are not 16-byte aligned");
  wdrz::LinearArgs a{};
  a.x = x;
  a.w = w;
  a.bias = bias;
  a.y = y;
  a.x_stride = x_stride;
  a.w_stride = w_stride;
  a.y_stride = y_stride;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.act = activation;
  hipError_t err = wdrz::launch_linear(dtype, a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

int wdrz_linear_partials(int dtype, const void* x, int64_t x_stride, const void* w, int64_t w_stride, float* partials,
                         int64_t M, int64_t N, int64_t K, int n_split, void* stream) {
  g_last_error.clear();
  if (dtype != WDRZ_BF16 && dtype != WDRZ_F16)
    return fail(dtype == WDRZ_F32 ? WDRZ_EUNSUPPORTED : WDRZ_EINVAL, "dtype %d: only WDRZ_BF16 / WDRZ_F16", dtype);
  if (n_split != 2 && n_split != 4) return fail(WDRZ_EUNSUPPORTED, "n_split %d is not 2 or 4", n_split);
  if (M < 0 || N <= 0 || K <= 0) return fail(WDRZ_EINVAL, "bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  if (K % (128 * n_split) != 0 || N % 8 != 0)
    return fail(WDRZ_EUNSUPPORTED, "K=%lld must be a multiple of 128 * n_split and N=%lld of 8", (long long)K,
                (long long)N);
  if (M > 65535 * 64 || N > (1 << 24) || K > (1 << 20) || M * N * n_split > ((int64_t)1 << 31))
    return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (M == 0) return WDRZ_OK;
  int rc;
  if ((rc = check_ptr("x", x)) || (rc = check_ptr("w", w)) || (rc = check_ptr("partials", partials))) return rc;
  if (x_stride < K || w_stride < K) return fail(WDRZ_EINVAL, "row strides shorter than the rows");
  if ((x_stride * 2) % 16 || (w_stride * 2) % 16) return fail(WDRZ_EINVAL, "row strides are not 16-byte aligned");
  wdrz::LinearArgs a{};
  a.x = x;
  a.w = w;
  a.x_stride = x_stride;
  a.w_stride = w_stride;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.part = partials;
  a.n_split = n_split;
  hipError_t err = wdrz::launch_linear(dtype, a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

int wdrz_add_layernorm_partials(int dtype, void* x, int64_t x_stride, const float* partials, int n_split,
                                const void* delta_bias, const void* weight, const void* bias, void* y,
                                int64_t y_stride, int64_t rows, int64_t n, float eps, void* stream) {
  g_last_error.clear();
  if (dtype != WDRZ_BF16 && dtype != WDRZ_F16)
    return fail(dtype == WDRZ_F32 ? WDRZ_EUNSUPPORTED : WDRZ_EINVAL, "dtype %d: only WDRZ_BF16 / WDRZ_F16", dtype);
  if (n_split != 2 && n_split != 4) return fail(WDRZ_EUNSUPPORTED, "n_split %d is not 2 or 4", n_split);
  if (rows < 0 || n <= 0 || n % 8 != 0)
    return fail(WDRZ_EINVAL, "bad sizes rows=%lld n=%lld (n must be a positive multiple of 8)", (long long)rows,
                (long long)n);
  if (n > 1536) return fail(WDRZ_EUNSUPPORTED, "n=%lld exceeds the supported 1536", (long long)n);
  if (rows > (1 << 24)) return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (!(eps >= 0.f)) return fail(WDRZ_EINVAL, "eps must be >= 0");
  if (rows == 0) return WDRZ_OK;
  int rc;
  if ((rc = check_ptr("x", x)) || (rc = check_ptr("partials", partials)) || (rc = check_ptr("delta_bias", delta_bias)) ||
      (rc = check_ptr("weight", weight)) || (rc = check_ptr("bias", bias)) || (rc = check_ptr("y", y)))
    return rc;
  if ((x_stride * 2) % 16 || (y_stride * 2) % 16) return fail(WDRZ_EINVAL, "row strides must be 16-byte aligned");
  if (rows > 1 && (x_stride < n || y_stride < n)) return fail(WDRZ_EINVAL, "row strides shorter than the rows");
  wdrz::AddLnArgs a{};
  a.x = x;
  a.weight = weight;
  a.bias = bias;
  a.y = y;
  a.rows = rows;
  a.n = (int)n;
  a.x_stride = x_stride;
  a.y_stride = y_stride;
  a.eps = eps;
  a.dpart = partials;
  a.n_part = n_split;
  a.dbias = delta_bias;
  hipError_t err = wdrz::launch_add_layernorm(dtype, a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

int wdrz_kv_fill(int dtype, const void* k_src, const void* v_src, const int64_t* src_strides, void* k_cache,
                 void* v_cache, const int64_t* cache_strides, const int64_t* slot_indices, int64_t B, int64_t T,
                 int64_t H, int64_t D, int64_t n_slots, int64_t Lmax, int64_t start_pos, void* stream) {
  g_last_error.clear();
  if (dtype != WDRZ_BF16 && dtype != WDRZ_F16)
    return fail(dtype == WDRZ_F32 ? WDRZ_EUNSUPPORTED : WDRZ_EINVAL, "dtype %d: only WDRZ_BF16 / WDRZ_F16", dtype);
  if (D != 64) return fail(WDRZ_EUNSUPPORTED, "head_dim %lld: only 64", (long long)D);
  if (B < 0 || T < 0 || H < 0 || n_slots < 0 || Lmax < 0 || start_pos < 0)
    return fail(WDRZ_EINVAL, "bad sizes B=%lld T=%lld H=%lld", (long long)B, (long long)T, (long long)H);
  if (start_pos + T > Lmax)
    return fail(WDRZ_EINVAL, "rows [%lld, %lld) exceed the cache length %lld", (long long)start_pos,
                (long long)(start_pos + T), (long long)Lmax);
  if (B > 65535 || H > 65535 || T > (1 << 24) || n_slots > (1 << 30)) return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (B == 0 || T == 0 || H == 0) return WDRZ_OK;
  if (!k_src || !v_src || !k_cache || !v_cache) return fail(WDRZ_EINVAL, "a K/V pointer is NULL");
  if (!src_strides || !cache_strides) return fail(WDRZ_EINVAL, "strides pointer is NULL");
  const void* ptrs[4] = {k_src, v_src, k_cache, v_cache};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 15) return fail(WDRZ_EINVAL, "K/V rows are not 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    if (((src_strides[i] * 2) & 15) || ((cache_strides[i] * 2) & 15))
      return fail(WDRZ_EINVAL, "K/V rows are not 16-byte aligned (strides)");
  wdrz::KvFillArgs a{};
  a.k_src = k_src;
  a.v_src = v_src;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  for (int i = 0; i < 3; ++i) {
    a.ss[i] = src_strides[i];
    a.cs[i] = cache_strides[i];
  }
  a.slots = slot_indices;
  a.B = (int)B;
  a.T = (int)T;
  a.H = (int)H;
  a.n_slots = (int)n_slots;
  a.start = (int)start_pos;
  hipError_t err = wdrz::launch_kv_fill(a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

int wdrz_median_filter(const float* x, int64_t x_stride, float* y, int64_t y_stride, int64_t rows, int64_t N,
                       int width, void* stream) {
  g_last_error.clear();
  if (width < 1 || (width > 1 && width % 2 == 0))
    return fail(WDRZ_EINVAL, "width %d must be 1 or odd (an even width makes the reference's reshape fail)", width);
  if (width / 2 > wdrz::kDtwMaxPad) return fail(WDRZ_EUNSUPPORTED, "width %d exceeds the supported 15", width);
  if (rows < 0 || N < 0) return fail(WDRZ_EINVAL, "bad sizes rows=%lld N=%lld", (long long)rows, (long long)N);
  if (N > (1 << 30) || rows * ((N + 2047) / 2048) > 0x7fffffff) return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (rows == 0 || N == 0) return WDRZ_OK;
  if (!x || !y) return fail(WDRZ_EINVAL, "x / y is NULL");
  if (x_stride < N || y_stride < N) return fail(WDRZ_EINVAL, "row strides shorter than the rows");
  wdrz::MedianArgs a{};
  a.x = x;
  a.xs = x_stride;
  a.y = y;
  a.ys = y_stride;
  a.rows = rows;
  a.N = (int)N;
  // a row no longer than the half width is returned as it is (dtw_align.py:66-67)
  a.pad = N <= width / 2 ? 0 : width / 2;
  hipError_t err = wdrz::launch_median_filter(a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

size_t wdrz_log_mel_workspace_size(int64_t B, int64_t n_mels) {
  if (B <= 0 || n_mels <= 0) return 0;
  return wdrz::logmel_workspace_bytes(B, n_mels);
}

int wdrz_log_mel(const float* audio, int64_t B, int64_t n_samples, int64_t audio_stride, float* out,
                 const int64_t* out_strides, int64_t n_mels, int64_t out_frames, void* workspace,
                 size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (B < 0 || n_mels <= 0) return fail(WDRZ_EINVAL, "bad sizes B=%lld n_mels=%lld", (long long)B, (long long)n_mels);
  if (n_mels > 128) return fail(WDRZ_EUNSUPPORTED, "n_mels=%lld exceeds the supported 128", (long long)n_mels);
  if (n_samples <= 200)
    return fail(WDRZ_EINVAL, "n_samples=%lld: the reflect padding of 200 needs more samples (as torch.stft)",
                (long long)n_samples);
  if (n_samples > (1 << 30) || B > 65535) return fail(WDRZ_EUNSUPPORTED, "sizes too large");
  if (!audio || !out || !out_strides) return fail(WDRZ_EINVAL, "audio / out / out_strides is NULL");
  if (audio_stride < n_samples && B > 1) return fail(WDRZ_EINVAL, "audio_stride is smaller than n_samples");
  if (out_strides[2] != 1) return fail(WDRZ_EINVAL, "out: frame stride must be 1");
  const int64_t n_frames = n_samples / 160;
  if (out_frames < 0) out_frames = n_frames;
  if (out_frames > (1 << 24)) return fail(WDRZ_EUNSUPPORTED, "out_frames too large");
  if (B == 0 || out_frames == 0) return WDRZ_OK;
  const size_t need = wdrz::logmel_workspace_bytes(B, n_mels);
  if (!workspace || workspace_bytes < need)
    return fail(WDRZ_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace ? workspace_bytes : 0);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(WDRZ_EINVAL, "workspace is not 256-byte aligned");
  wdrz::LogMelArgs a{};
  a.audio = audio;
  a.audio_stride = audio_stride;
  a.out = out;
  a.os[0] = out_strides[0];
  a.os[1] = out_strides[1];
  a.B = (int)B;
  a.n_samples = (int)n_samples;
  a.n_mels = (int)n_mels;
  a.n_frames = (int)n_frames;
  a.out_frames = (int)out_frames;
  hipError_t err = wdrz::launch_logmel(a, workspace, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

size_t wdrz_dtw_prep_workspace_size(int64_t B, int64_t H, int64_t T, int64_t A) {
  if (B <= 0 || H <= 0 || T <= 0 || A <= 0) return 0;
  return wdrz::dtw_workspace_bytes(B, H, T, A);
}

int wdrz_dtw_prep(const float* weights, const int64_t* w_strides, const int32_t* actual_lens,
                  const int32_t* audio_caps, float* out, const int64_t* out_strides, int64_t B, int64_t H,
                  int64_t T, int64_t A, int64_t C, int medfilt_width, void* workspace, size_t workspace_bytes,
                  void* stream) {
  g_last_error.clear();
  if (!weights) return fail(WDRZ_EINVAL, "weights is NULL");
  if (!w_strides) return fail(WDRZ_EINVAL, "strides pointer is NULL");
  if (w_strides[3] != 1) return fail(WDRZ_EINVAL, "weights: last stride must be 1");
  wdrz::DtwArgs a{};
  int rc = dtw_common_args(actual_lens, audio_caps, out, out_strides, B, H, T, A, C, medfilt_width, workspace,
                           workspace_bytes, &a);
  if (rc == -1) return WDRZ_OK;
  if (rc != WDRZ_OK) return rc;
  a.w = weights;
  for (int i = 0; i < 3; ++i) a.ws[i] = w_strides[i];
  hipError_t err = wdrz::launch_dtw_prep(a, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

int wdrz_dtw_attention_prep(int dtype, const void* const* q_heads, const int64_t* q_strides,
                            const void* const* k_heads, const int64_t* k_strides, float scale,
                            const int32_t* actual_lens, const int32_t* audio_caps, float* out,
                            const int64_t* out_strides, int64_t B, int64_t H, int64_t T, int64_t A, int64_t D,
                            int64_t C, int medfilt_width, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (!(scale > 0.f) || scale != scale) return fail(WDRZ_EINVAL, "scale must be a positive finite number");
  if (A > wdrz::kDtwQkMaxA)
    return fail(WDRZ_EUNSUPPORTED, "A=%lld audio rows exceed the supported %d", (long long)A, wdrz::kDtwQkMaxA);
  wdrz::DtwQkArgs q{};
  int rc = dtw_qk_heads(dtype, q_heads, q_strides, k_heads, k_strides, H, D, &q);
  if (rc != WDRZ_OK) return rc;
  q.scale2 = scale * scale;
  if (A > 0 && ((A - 1) * k_strides[1] + D) * 2 >= (int64_t(1) << 32))
    return fail(WDRZ_EUNSUPPORTED, "one batch row of keys spans more than 4 GiB");
  wdrz::DtwArgs a{};
  rc = dtw_common_args(actual_lens, audio_caps, out, out_strides, B, H, T, A, C, medfilt_width, workspace,
                       workspace_bytes, &a);
  if (rc == -1) return WDRZ_OK;
  if (rc != WDRZ_OK) return rc;
  hipError_t err = wdrz::launch_dtw_qk_prep(dtype, a, q, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(WDRZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return WDRZ_OK;
}

}  // extern "C"
