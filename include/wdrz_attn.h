/*
 * wdrz_attn.h — C ABI of libwdrz_attn.so, the MI355X (gfx950) attention hot path of
 * WhisperDRZ.
 *
 * Two entry points replace the reference's two attention seams:
 *
 *   wdrz_attn_fwd      replaces F.scaled_dot_product_attention as called from
 *                      MultiHeadAttention.qkv_attention (src/whisperdrz/model.py:276-298,
 *                      the SDPA call itself at model.py:288-296): encoder self-attention
 *                      (non-causal, L=1500) and the uncached decoder (causal, top-left).
 *
 *   wdrz_attn_kvcache  replaces flash_attn_with_kvcache / its torch fallback
 *                      _sdpa_attn_with_kvcache (src/whisperdrz/model.py:20-95), as called from
 *                      MultiHeadAttention.forward_flash (model.py:336-344 cross, 349-359 self):
 *                      decoder cached self-attention with fused in-place K/V append, decoder
 *                      cross-attention, and multi-token (prefill / draft-verify) queries.
 *
 * Conventions
 *   - All pointers are device pointers owned by the caller. The library never allocates,
 *     frees or synchronises, and never reads device memory from the host, so every call is
 *     safe inside hipGraph stream capture.
 *   - Strides are in ELEMENTS (not bytes). The last (head_dim) dimension must be contiguous
 *     (stride 1); every other stride and every base pointer must be 16-byte aligned.
 *   - head_dim must be 64 (every Whisper size uses 64).
 *   - `stream` is a hipStream_t (0 = the null stream).
 *   - Every function returns 0 on success or a WDRZ_E* code; wdrz_last_error() then returns a
 *     thread-local message naming the offending argument.
 */
#ifndef WDRZ_ATTN_H
#define WDRZ_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (the reference runs fp16 on GPU, model.py:769-770; fp32 on CPU,
 * transcriber.py:662-663; bf16 is the build's headline type). */
#define WDRZ_F32 0
#define WDRZ_F16 1
#define WDRZ_BF16 2

/* Status codes. */
#define WDRZ_OK 0
#define WDRZ_EINVAL 1       /* bad argument (shape, stride, alignment, null pointer) */
#define WDRZ_EUNSUPPORTED 2 /* valid for the reference but not implemented (e.g. D != 64) */
#define WDRZ_ELAUNCH 3      /* the HIP launch itself failed */
#define WDRZ_EWORKSPACE 4   /* workspace missing or too small */

/* Thread-local message for the last failing call on this thread ("" if none). */
const char* wdrz_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int wdrz_abi_version(void);

/* Hash of the sources the library was built from (kernels, C-ABI layer, this header, build
 * flags). No counterpart in the reference: the Python loader compares it with the tree it runs
 * from and refuses a library built from other sources. */
const char* wdrz_build_id(void);

/*
 * Dense scaled-dot-product attention, O = softmax(scale * Q K^T [+ causal mask]) V, per (b, h).
 *
 * Replaces: F.scaled_dot_product_attention(q, k, v, is_causal=..., attn_mask=None,
 *           scale=1/8, dropout_p=0) at src/whisperdrz/model.py:288-296.
 *
 * q: [B, H, Lq, D], k, v: [B, H, Lk, D], o: [B, H, Lq, D], each described by 4 strides in
 * [B, H, L, D] order (the reference passes rearranged, non-contiguous views of the
 * [B, T, H*D] projection output, model.py:282-284, so strides are honoured).
 * causal != 0 applies torch's is_causal mask (top-left aligned: query i sees keys j <= i).
 * dtype: WDRZ_BF16 / WDRZ_F16 use the bf16 / fp16 MFMA kernels; WDRZ_F32 the fp32 MFMA kernel
 *        (v_mfma_f32_32x32x2_f32, fp32 accumulation).
 */
int wdrz_attn_fwd(int dtype, const void* q, const void* k, const void* v, void* o, int64_t B,
                  int64_t H, int64_t Lq, int64_t Lk, int64_t D, const int64_t* q_strides,
                  const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
                  float scale, int causal, void* stream);

/*
 * Workspace (bytes) that wdrz_attn_kvcache needs for these sizes. 0 means none is needed:
 * enough rows to fill the chip (B * ceil(sq / 8) * H >= 1024), or sq >= 40 (those calls never
 * split their keys).
 * No counterpart in the reference: flash-attn allocates its split-KV scratch internally; this
 * library leaves allocation to the caller so calls can be captured into a hipGraph.
 */
size_t wdrz_attn_kvcache_workspace_size(int64_t B, int64_t sq, int64_t H, int64_t D,
                                        int64_t Lmax);

/*
 * Attention against a slot KV cache.
 *
 * Replaces: flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, cache_seqlens=None,
 *           cache_batch_idx=None, softmax_scale=None, causal=False)
 *           (dispatcher src/whisperdrz/model.py:88-95; semantics of the torch fallback
 *           _sdpa_attn_with_kvcache, model.py:20-76).
 *
 * q:        [B, sq, H, D]                      strides q_strides[4]
 * k_cache,  [n_slots, Lmax, H, D]              strides kc_strides[4], vc_strides[4]
 * v_cache
 * k_new,    [B, sq, H, D] or both NULL         strides kn_strides[4], vn_strides[4]
 * v_new
 * cache_seqlens   int32 [B]: pre-append length per batch row (required iff k_new given)
 * cache_batch_idx int32 [B]: batch row -> slot (NULL = identity; must be < n_slots)
 * o:        [B, sq, H, D], same dtype as q     strides o_strides[4]
 *
 * Self-attention (k_new != NULL), model.py:49-63:
 *   k_new[b, t], v_new[b, t] are written IN PLACE to cache row cache_seqlens[b] + t of slot
 *   cache_batch_idx[b]; query t attends keys j <= cache_seqlens[b] + t (bottom-right causal).
 *   cache_seqlens itself is NOT modified (the caller bumps it, model.py:602-607).
 * Cross-attention (k_new == NULL), model.py:64-67: non-causal attention over all Lmax rows
 *   (cache_seqlens is ignored, as in the fallback).
 * `causal` is accepted for signature parity; as in the fallback, the mask is decided by
 *   whether k_new is given.
 * Repeated cache_batch_idx entries with k_new given follow the reference fallback's order
 *   (model.py:51-57): a cache position ends up holding the new row of the LAST batch row whose
 *   region [cache_seqlens, cache_seqlens + sq) covers it, and every row attends over the cache
 *   after all appends.
 * workspace: device buffer of at least wdrz_attn_kvcache_workspace_size(...) bytes, 256-byte
 *   aligned (may be NULL when that is 0). It holds per-row arrival counters and partials and
 *   must be all-zero when a call starts: zero-fill the buffer once after allocating it; every
 *   completed call leaves it all-zero again, whatever the shapes of earlier calls. Concurrent
 *   calls must not share a workspace.
 */
int wdrz_attn_kvcache(int dtype, const void* q, void* k_cache, void* v_cache, const void* k_new,
                      const void* v_new, const int32_t* cache_seqlens,
                      const int32_t* cache_batch_idx, void* o, int64_t B, int64_t sq, int64_t H,
                      int64_t D, int64_t n_slots, int64_t Lmax, const int64_t* q_strides,
                      const int64_t* kc_strides, const int64_t* vc_strides,
                      const int64_t* kn_strides, const int64_t* vn_strides,
                      const int64_t* o_strides, float softmax_scale, int causal, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * Attention against a slot KV cache without any allocation: wdrz_attn_kvcache with its split-KV
 * workspace taken from a static device array of WDRZ_NOALLOC_SCRATCH_BYTES per GPU.
 *
 * No counterpart in the reference. For callers that cannot allocate: code under hipGraph
 * capture without an allocator, tight serving loops, harnesses that forbid hipMalloc. It calls
 * no hipMalloc / hipFree and no allocating library routine.
 *
 * Arguments and semantics as wdrz_attn_kvcache, without workspace / workspace_bytes.
 * Limit: calls whose workspace (wdrz_attn_kvcache_workspace_size) exceeds
 * WDRZ_NOALLOC_SCRATCH_BYTES are rejected with WDRZ_EUNSUPPORTED (the split plan never asks
 * for more than ~4.33 MB at head_dim 64). The array is set up (address taken, cleared by a
 * kernel on `stream`) on the first call on each device and kept until the process ends. The
 * array is zero when the code object loads (a zero-initialised device global) and every completed
 * call leaves it zero, so a first call made under graph capture, whose clearing kernel is then
 * recorded into the graph rather than run, still starts from zero, both in eager calls made
 * before the first replay and in every replay.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU race; serialise
 * them or use wdrz_attn_kvcache with separate workspaces.
 */
#define WDRZ_NOALLOC_SCRATCH_BYTES ((size_t)4718592) /* 4.5 MiB */
int wdrz_attn_kvcache_noalloc(int dtype, const void* q, void* k_cache, void* v_cache,
                              const void* k_new, const void* v_new, const int32_t* cache_seqlens,
                              const int32_t* cache_batch_idx, void* o, int64_t B, int64_t sq,
                              int64_t H, int64_t D, int64_t n_slots, int64_t Lmax,
                              const int64_t* q_strides, const int64_t* kc_strides,
                              const int64_t* vc_strides, const int64_t* kn_strides,
                              const int64_t* vn_strides, const int64_t* o_strides,
                              float softmax_scale, int causal, void* stream);

/*
 * The MLP input projection of the decode step with its activation: Y = act(X W^T + b).
 *
 * Replaces: the first two modules of ResidualAttentionBlock.mlp, Linear(n_state, 4 n_state)
 *           and nn.GELU() (src/whisperdrz/model.py:388-391, applied at model.py:434): the
 *           library GEMM with bias, its rounding to the 16-bit type, then the exact (erf) GELU
 *           and its rounding, in one launch.
 * x: [M, K] rows (stride x_stride), w: [N, K] rows (the Linear's weight, stride w_stride),
 * bias: [N] or NULL, y: [M, N] rows (stride y_stride); 16-bit types, fp32 accumulation.
 * activation: 0 none, 1 GELU (0.5 v (1 + erf(v / sqrt 2))). K % 128 == 0, N % 8 == 0,
 * pointers and row strides 16-byte aligned. Sized for the decode step's few rows (M <= 64 per
 * workgroup row block; any M works).
 */
int wdrz_linear(int dtype, const void* x, int64_t x_stride, const void* w, int64_t w_stride,
                const void* bias, void* y, int64_t y_stride, int64_t M, int64_t N, int64_t K,
                int activation, void* stream);

/*
 * Residual add + LayerNorm of the decode step.
 *
 * Replaces: the residual add closing a sub-layer and the LayerNorm opening the next
 *           (src/whisperdrz/model.py:420-433, ResidualAttentionBlock.forward_flash; the final
 *           ln before the logits, model.py:609-613; LayerNorm model.py:195-200 in eval mode).
 * x:      16-bit rows [rows, n], row stride x_stride; when delta != NULL it is updated in place to
 *         x + delta (rounded to the storage type, as torch's add), the new residual.
 * y:      LayerNorm(x) rows, fp32 statistics, eps, affine weight / bias (16-bit, [n]).
 * n a multiple of 8, <= 4096; 16-byte aligned pointers and row strides.
 */
int wdrz_add_layernorm(int dtype, void* x, int64_t x_stride, const void* delta,
                       int64_t delta_stride, const void* weight, const void* bias, void* y,
                       int64_t y_stride, int64_t rows, int64_t n, float eps, void* stream);

/*
 * The MLP output projection of the decode step, split along K (the first half of a pair with
 * wdrz_add_layernorm_partials).
 *
 * Replaces: the last module of ResidualAttentionBlock.mlp, Linear(4 n_state, n_state)
 *           (src/whisperdrz/model.py:388-391, applied at model.py:434), whose K = 4 n_state is
 *           long and whose output is narrow: the library GEMM runs few workgroups for it.
 * x: [M, K] rows (stride x_stride), w: [N, K] rows (stride w_stride), 16-bit types.
 * partials: fp32 [n_split][M][N], contiguous: split z holds sum over k in [z K / n_split,
 * (z + 1) K / n_split) of x[m, k] w[n, k]; no bias, no rounding. n_split 2 or 4,
 * K % (128 n_split) == 0, N % 8 == 0, pointers and row strides 16-byte aligned.
 */
int wdrz_linear_partials(int dtype, const void* x, int64_t x_stride, const void* w, int64_t w_stride,
                         float* partials, int64_t M, int64_t N, int64_t K, int n_split, void* stream);

/*
 * Residual add + LayerNorm with the delta given as a Linear's split-K partials (the second half
 * of the pair with wdrz_linear_partials).
 *
 * Replaces: x = x + mlp(mlp_ln(x)) and the LayerNorm that follows (src/whisperdrz/model.py:434
 *           then 420 of the next block, or the final ln, model.py:609-613): the Linear's output
 *           delta = round(sum over z of partials[z] + delta_bias), rounded to the 16-bit type
 *           as the library GEMM's output is; then x = round(x + delta) in place and
 *           y = LayerNorm(x) as wdrz_add_layernorm computes it.
 * partials: fp32 [n_split][rows][n] contiguous; delta_bias: the Linear's bias [n] (16-bit);
 * n_split 2 or 4; n a multiple of 8, <= 1536; 16-byte aligned pointers and row strides.
 */
int wdrz_add_layernorm_partials(int dtype, void* x, int64_t x_stride, const float* partials,
                                int n_split, const void* delta_bias, const void* weight,
                                const void* bias, void* y, int64_t y_stride, int64_t rows,
                                int64_t n, float eps, void* stream);

/*
 * Greedy sampling with the decode step's token constraints.
 *
 * Replaces: decode_batch's sampling tail (src/whisperdrz/decoding.py:1729-1761):
 *           masked = logits + (-65504 where blocked[row, v]); where penalty[row, v]:
 *           masked > 0 ? masked / 1.2 : masked * 1.2; out[row] = argmax (temperature 0,
 *           sample_logits decoding.py:854-855). Every step rounds to the logits' type as the
 *           torch ops do; ties go to the lowest index, as torch.argmax.
 * logits: [rows, V] (f32 / f16 / bf16), row stride logits_stride (elements).
 * blocked, penalty: bool [rows, V] as bytes (row strides in bytes), either may be NULL.
 * out: int64 [rows].
 */
int wdrz_masked_argmax(int dtype, const void* logits, int64_t logits_stride,
                       const uint8_t* blocked, int64_t blocked_stride, const uint8_t* penalty,
                       int64_t penalty_stride, int64_t* out, int64_t rows, int64_t V, void* stream);

/*
 * Workspace (bytes) for wdrz_log_mel: the [202, n_mels] filterbank and one maximum per window.
 * No counterpart in the reference (torchaudio keeps the filterbank in a module buffer).
 */
size_t wdrz_log_mel_workspace_size(int64_t B, int64_t n_mels);

/*
 * Whisper log-mel spectrogram of B waveforms.
 *
 * Replaces: LogMelSpectrogram.forward / _process_single_audio (src/whisperdrz/audio.py:108-156),
 *           which the reference computes on the CPU per 30-s window (transcriber.py:1091-1092).
 *           torch.stft(n_fft 400, hop 160, periodic Hann, center, reflect) -> |X|^2 without the
 *           last frame -> slaney mel filterbank -> log10(max(., 1e-10)) -> max(., max - 8) over
 *           each window -> (x + 4) / 4 -> pad with -1.5 or truncate to out_frames.
 *
 * audio:      fp32 [B, n_samples], row stride audio_stride (elements); n_samples > 200.
 * out:        fp32 [B, n_mels, out_frames], strides out_strides[3] (frame stride 1).
 * out_frames: the reference's target_frames, or -1 for n_samples / 160 frames (no padding).
 * n_mels <= 128 (Whisper uses 80 or 128). workspace: wdrz_log_mel_workspace_size(B, n_mels)
 * bytes, 256-byte aligned; no state is kept in it between calls.
 */
int wdrz_log_mel(const float* audio, int64_t B, int64_t n_samples, int64_t audio_stride,
                 float* out, const int64_t* out_strides, int64_t n_mels, int64_t out_frames,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Raw cross-attention scores of the DTW alignment heads.
 *
 * Replaces: CrossAttnCapture.compute_attention(head_mask) (src/whisperdrz/dtw_align.py:553-586):
 *           S[b, h, t, a] = sum_d (Q_h[b, t, d] * scale) * (K_h[b, a, d] * scale), no softmax,
 *           scale = head_dim^-0.25 (dtw_align.py:561), fp32 result.
 *
 * q_heads[h]: device pointer to head h's query slice of the captured cross_attn.query output of
 *             its layer (e.g. q_out[layer] + head*64 elements); rows (b, t) at
 *             q_heads[h] + b*q_strides[0] + t*q_strides[1], the head_dim elements contiguous
 *             (q_strides[2] == 1). Same for k_heads / k_strides over the 1500 audio rows.
 *             q_heads and k_heads are HOST arrays of H device pointers; all heads share the
 *             strides. bf16 or fp16 (the reference's GPU model dtype); 16-byte aligned.
 * out:        fp32 [B, H, T, A], strides out_strides[4] (last one 1). The reference returns
 *             [H, T, A] when B == 1; callers lift it back to 4-D (dtw_align.py:1185-1187).
 * H <= 32, head_dim 64.
 */
int wdrz_dtw_qk(int dtype, const void* const* q_heads, const int64_t* q_strides,
                const void* const* k_heads, const int64_t* k_strides, float* out,
                const int64_t* out_strides, int64_t B, int64_t H, int64_t T, int64_t A,
                int64_t D, float scale, void* stream);

/*
 * Workspace (bytes) that wdrz_dtw_prep needs: one (max, 1/sum) pair per score row and one
 * (mean, 1/std) pair per score column, 8 * B*H*(T + A) bytes plus alignment.
 * No counterpart in the reference: torch allocates the intermediates of _dtw_prep_batch itself.
 */
size_t wdrz_dtw_prep_workspace_size(int64_t B, int64_t H, int64_t T, int64_t A);

/*
 * DTW alignment prep of the cross-attention scores.
 *
 * Replaces: _dtw_prep_batch(full_weights, actual_lens, audio_caps, medfilt_width)
 *           (src/whisperdrz/dtw_align.py:700-753) up to its device->host copy, with the median
 *           filter it calls (median_filter, dtw_align.py:156-167: the Triton kernel at
 *           dtw_align.py:87-155 on GPU, the sort-based filter at dtw_align.py:65-78 elsewhere).
 *
 * weights:     fp32 [B, H, T, A] raw Q K^T of the H alignment heads (CrossAttnCapture.
 *              compute_attention, dtw_align.py:553-586), strides w_strides[4] in elements,
 *              last one 1 (rows that start 16-byte aligned are read with 16-byte loads).
 * actual_lens: int32 [B] valid text rows per batch row (the column statistics use rows
 *              t < actual_lens[b] and divide by actual_lens[b]; every row is normalised).
 * audio_caps:  int32 [B] valid audio columns per batch row (columns >= cap get softmax 0).
 * out:         fp32 [B, T, C], strides out_strides[3] (last one 1). C must be
 *              min(max(audio_caps), A) — the reference's slice [:, :, :max_audio_cap] — as the
 *              library does not read the device-side caps on the host.
 * medfilt_width: 1 (no filter) or odd <= 15; reflect padding; skipped when A <= width / 2.
 * workspace:   device buffer of wdrz_dtw_prep_workspace_size(B, H, T, A) bytes, 256-byte aligned;
 *              no state is kept in it between calls.
 * T <= 512 (Whisper's text context is 448). A batch row with actual_lens[b] == 0 or
 * audio_caps[b] == 0 gives NaN everywhere, as the reference's 0/0 does. Inputs must be finite.
 */
int wdrz_dtw_prep(const float* weights, const int64_t* w_strides, const int32_t* actual_lens,
                  const int32_t* audio_caps, float* out, const int64_t* out_strides, int64_t B,
                  int64_t H, int64_t T, int64_t A, int64_t C, int medfilt_width, void* workspace,
                  size_t workspace_bytes, void* stream);

/*
 * Fused DTW prep straight from the captured projections: wdrz_dtw_qk followed by wdrz_dtw_prep,
 * without the [B, H, T, A] fp32 score tensor ever being written to or read from memory.
 *
 * Replaces: full_weights = cap.compute_attention(head_mask) and _dtw_prep_batch(full_weights,
 *           actual_lens, audio_caps) (src/whisperdrz/dtw_align.py:1184 and 1197; the functions
 *           at dtw_align.py:553-586 and 700-753) up to the device->host copy.
 *
 * q_heads / k_heads / strides / scale / dtype: as for wdrz_dtw_qk (H <= 32, head_dim 64).
 * actual_lens / audio_caps / out / C / medfilt_width: as for wdrz_dtw_prep.
 * workspace:  device buffer of wdrz_dtw_prep_workspace_size(B, H, T, A) bytes, 256-byte aligned.
 * A <= 1536 (Whisper's 1500 audio frames); T <= 512. Each score is computed identically in the
 * statistics pass and the filter pass, so the result equals wdrz_dtw_prep applied to
 * wdrz_dtw_qk's output up to the fp32 rounding of the summation order of the dot products.
 */
int wdrz_dtw_attention_prep(int dtype, const void* const* q_heads, const int64_t* q_strides,
                            const void* const* k_heads, const int64_t* k_strides, float scale,
                            const int32_t* actual_lens, const int32_t* audio_caps, float* out,
                            const int64_t* out_strides, int64_t B, int64_t H, int64_t T,
                            int64_t A, int64_t D, int64_t C, int medfilt_width, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Projected K/V rows into the slot caches:
 *   k_cache[slot_indices[b], start_pos + t, h, :] = k_src[b, t, h, :]   (and v), t < T.
 *
 * Replaces: FlashKVCache.prefill(k, v, start_pos, slot_indices) and
 *           FlashKVCache.set_cross_attention(k, v, slot_indices) (src/whisperdrz/model.py:150-183),
 *           the cache writes of prefill_flash's cross fill (model.py:851-862); the callers keep
 *           the seq_lens / cross_attn_len bookkeeping.
 *
 * k_src / v_src: [B, T, H, 64] 16-bit, element strides src_strides[3] of b, t, h (head_dim
 *                contiguous; e.g. the key / value halves of one fused projection output).
 * k_cache / v_cache: [n_slots, Lmax, H, 64], strides cache_strides[3] of slot, position, head
 *                (any order: head-major storage viewed slot-major works).
 * slot_indices:  device int64 [B], or NULL for slot b. Ids outside [0, n_slots) are skipped.
 * Rows 16-byte aligned; start_pos + T <= Lmax. Each element is written once (duplicate slot ids
 * race, as the reference's index_put does).
 */
int wdrz_kv_fill(int dtype, const void* k_src, const void* v_src, const int64_t* src_strides,
                 void* k_cache, void* v_cache, const int64_t* cache_strides,
                 const int64_t* slot_indices, int64_t B, int64_t T, int64_t H, int64_t D,
                 int64_t n_slots, int64_t Lmax, int64_t start_pos, void* stream);

/*
 * Median filter along the last axis, reflect padding.
 *
 * Replaces: median_filter(x, width) (src/whisperdrz/dtw_align.py:156-167: the Triton kernel of
 *           dtw_align.py:87-155 on GPU, the sort-based _median_filter_sort of dtw_align.py:65-78
 *           elsewhere), for fp32 rows: y[r, c] = median(x[r, c - width/2 .. c + width/2]).
 * x, y:   fp32 [rows, N], row strides in elements (last stride 1); y may not alias x.
 * width:  1 or odd <= 15. A row with N <= width/2 is copied unchanged (dtw_align.py:66-67).
 * Inputs must be finite (NaN ordering is not torch.sort's).
 */
int wdrz_median_filter(const float* x, int64_t x_stride, float* y, int64_t y_stride, int64_t rows,
                       int64_t N, int width, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WDRZ_ATTN_H */
