// wdrz_launch.h — internal (C++) launch interface between the C-ABI layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wdrz {

// Split-KV attention over a key/value store, used both for the cached decoder paths and for
// the fp32 dense path. Strides are in BYTES; the last (head_dim) dimension is contiguous.
//
// Query row (b, t, h) lives at q + b*qs[0] + t*qs[1] + h*qs[2] (same for o, k_new, v_new).
// Key j of batch row b, head h lives at kv + slot(b)*kvs[0] + j*kvs[1] + h*kvs[2].
struct KvArgs {
  const char* q;
  char* kc;
  char* vc;
  const char* kn;  // k_new (nullptr: no append)
  const char* vn;
  const int32_t* seqlens;  // pre-append lengths (required with k_new)
  const int32_t* bidx;     // batch row -> slot (nullptr: identity)
  char* o;
  float* ws_part;  // split partials (split mode with n_splits > 1)
  int* ws_count;   // per-row arrival counters, zero between calls
  int B, sq, H, Lk, n_slots, n_qblocks, n_splits, split_len;
  int mq_rows;  // 16: query blocks of 16 rows on the multi-query MFMA kernel; 0: blocks of 8 (or one block)
  int64_t qs[3], kcs[3], vcs[3], kns[3], vns[3], os[3];
  float c;  // softmax scale * log2(e)
};

// Split count and keys per split for `units` = B*n_qblocks*H rows over Lk keys.
// Depends only on sizes, so the workspace size can be queried without data.
void kv_split_plan(int64_t units, int64_t Lk, int* n_splits, int* split_len);
// Workspace when n_splits > 1: per-row int32 counters (zero between calls), then partials.
size_t kv_workspace_bytes(int64_t units, int64_t sq_blk, int n_splits);
void kv_workspace_layout(void* ws, int64_t units, KvArgs* a);

// Launch the attention kernel: one workgroup per (row, key split); with n_splits > 1 the
// partials merge in-launch through the workspace. dtype: 0 f32, 1 f16, 2 bf16.
hipError_t launch_kv_attn(int dtype, const KvArgs& a, hipStream_t stream);
// Many-query cached attention (16-bit, sq >= kPrefillMinSq): 256-query MFMA blocks. Self (new
// rows given): causal, keys below cache_seqlens from the slot and the rest from k_new / v_new, the
// new rows appended. Cross (no new rows): all Lk cache rows, nothing appended.
constexpr int kPrefillMinSq = 40;
hipError_t launch_kv_prefill(int dtype, const KvArgs& a, hipStream_t stream);

// Dense MFMA attention (bf16 / fp16). Strides in ELEMENTS in [B, H, L, D] order.
struct DenseArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int B, H, Lq, Lk, causal;
  int bh0;                             // first (b * H + h) of a dense_split_kernel launch
  int64_t qs[3], ks[3], vs[3], os[3];  // b, h, l strides
  float c;                             // softmax scale * log2(e)
  // dense_pipe_kernel only: K/V of batch row b at slot slot[b] (nullptr: b); a slot outside
  // [0, n_slots) gives that row's output as NaN, as the cached-attention kernels do
  const int32_t* slot = nullptr;
  int n_slots = 0;
};
hipError_t launch_dense_mfma(int dtype, const DenseArgs& a, hipStream_t stream);
// The same on the fp32 matrix cores (fp32 inputs and output; causal = top-left).
hipError_t launch_dense_f32(const DenseArgs& a, hipStream_t stream);

// DTW alignment prep over fp32 scores W [B, H, T, A] (strides in ELEMENTS, last one 1).
constexpr int kDtwMaxRows = 512;  // T limit (Whisper's text context is 448)
constexpr int kDtwMaxPad = 7;     // median width <= 15
struct DtwArgs {
  const float* w;
  const int32_t* lens;  // [B] valid text rows
  const int32_t* caps;  // [B] valid audio columns
  float* out;           // [B, T, C]
  float2* rs;           // workspace: per-row (max*log2e, 1/sum)
  float2* cs;           // workspace: per-column (mean, 1/std), row pitch cpitch
  float2* part;         // workspace: per-64-row-chunk column partials (mean, M2), pitch cpitch
  int B, H, T, A, C, pad;
  int cpitch;   // A rounded up to a multiple of 4
  int rc_rows;  // rows per chunk of the fused statistics pass
  int vec;     // rows of W start 16-byte aligned (set by the launcher)
  int nt_b;    // statistics pass: batch rows below this are read nontemporally (set by the launcher)
  int64_t ws[3];  // W strides b, h, t
  int64_t os[2];  // out strides b, t
};
// Raw Q K^T of the alignment heads (bf16 / fp16 in, fp32 out). Q head h: rows (b, t) at
// q[h] + b*qs[0] + t*qs[1] (elements, head dims contiguous); K likewise with a for t.
constexpr int kDtwMaxHeads = 32;
struct DtwQkArgs {
  const void* q[kDtwMaxHeads];
  const void* k[kDtwMaxHeads];
  float* out;  // [B, H, T, A]
  int B, H, T, A;
  int64_t qs[2], ks[2];  // b, row strides
  int64_t os[3];         // b, h, t strides of out
  float scale2;          // (head_dim^-0.25)^2 as the product of the two fp32 scales
  int vec;               // out rows 16-byte aligned (set by the launcher)
};
hipError_t launch_dtw_qk(int dtype, DtwQkArgs a, hipStream_t stream);

// Residual add + LayerNorm over 16-bit rows (strides in elements).
struct AddLnArgs {
  void* x;            // residual rows, updated in place to x + delta (when delta is given)
  const void* delta;  // nullptr: LayerNorm of x only
  const void* weight;
  const void* bias;
  void* y;            // LayerNorm output rows
  int64_t rows;
  int n;
  int64_t x_stride, d_stride, y_stride;
  float eps;
  // delta given as fp32 split-K partials [n_part][rows][n] of a Linear plus its 16-bit bias:
  // delta = round(sum of the partials + bias), as the Linear's output (used when dpart != nullptr)
  const float* dpart = nullptr;
  int n_part = 0;
  const void* dbias = nullptr;
};
hipError_t launch_add_layernorm(int dtype, const AddLnArgs& a, hipStream_t stream);

// Masked greedy sampling over logits rows (strides in elements / bytes for the masks).
// Rows of projected K/V into the slot caches (kv_fill.hip): cache[slot[b], start + t, h, :] =
// src[b, t, h, :] for K and V; 16-bit elements, head_dim 64, strides in elements.
struct KvFillArgs {
  const void* k_src;
  const void* v_src;
  int64_t ss[3];  // source strides of b, t, h (the head_dim is contiguous)
  void* k_cache;
  void* v_cache;
  int64_t cs[3];  // cache strides of slot, position, head
  const int64_t* slots;  // [B] slot of each batch row, or null for slot b
  int B, T, H;
  int n_slots, start;
};
hipError_t launch_kv_fill(const KvFillArgs& a, hipStream_t stream);

// Median filter along rows (dtw_prep.hip): y[r, c] = median of x[r, c-pad .. c+pad], reflected.
struct MedianArgs {
  const float* x;
  int64_t xs;
  float* y;
  int64_t ys;
  int64_t rows;
  int N, pad;
  int vec;  // rows 16-byte aligned: vector loads / stores
};
hipError_t launch_median_filter(const MedianArgs& a, hipStream_t stream);

struct ArgmaxArgs {
  const void* logits;
  int64_t l_stride;
  const uint8_t* blocked;  // bool [rows, V] or nullptr
  int64_t m_stride;
  const uint8_t* penalty;  // bool [rows, V] or nullptr
  int64_t p_stride;
  int64_t* out;
  int rows, V;
};
hipError_t launch_masked_argmax(int dtype, const ArgmaxArgs& a, hipStream_t stream);

// Y[M, N] = act(X[M, K] W[N, K]^T + b[N]) in 16-bit types (act 0: none, 1: GELU, erf form).
// Strides in elements (rows); K % 128 == 0, N % 8 == 0, rows 16-byte aligned.
struct LinearArgs {
  const void* x;
  const void* w;
  const void* bias;  // nullptr: no bias
  void* y;
  int64_t x_stride, w_stride, y_stride;
  int M, N, K, act;
  float* part = nullptr;  // split-K form: fp32 partials [n_split][M][N] instead of y
  int n_split = 1;
};
hipError_t launch_linear(int dtype, const LinearArgs& a, hipStream_t stream);

// Log-mel front end over fp32 waveforms [B, n_samples] (row stride audio_stride elements).
struct LogMelArgs {
  const float* audio;
  int64_t audio_stride;
  float* out;         // [B, n_mels, out_frames], frames contiguous
  int64_t os[2];      // b, mel strides of out
  float* fb;          // workspace: [202, n_mels] filterbank
  float* tables;      // workspace: cos(2 pi j / 400), then the periodic Hann window
  uint32_t* gmax;     // workspace: [B] ordered-encoded window maxima
  int B, n_samples, n_mels, n_frames, out_frames;
};
size_t logmel_workspace_bytes(int64_t B, int64_t n_mels);
hipError_t launch_logmel(LogMelArgs a, void* ws, hipStream_t stream);

size_t dtw_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A);
// The prep with the scores computed from the heads' Q / K inside both passes (A <= 1536).
constexpr int kDtwQkMaxA = 1536;
hipError_t launch_dtw_qk_prep(int dtype, DtwArgs a, const DtwQkArgs& q, hipStream_t stream);
void dtw_workspace_layout(void* ws, DtwArgs* a);
hipError_t launch_dtw_prep(DtwArgs a, hipStream_t stream);

// Sets the thread-local message wdrz_last_error() returns and returns `code` (C-ABI layer).
int set_last_error(int code, const char* fmt, ...);

}  // namespace wdrz
