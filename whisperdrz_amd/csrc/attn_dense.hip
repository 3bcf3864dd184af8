// attn_dense.hip — flash-style dense attention on CDNA4 bf16/fp16 MFMA (gfx950).
//
// Replaces F.scaled_dot_product_attention at reference src/whisperdrz/model.py:288-296
// (encoder self-attention, [B, 20, 1500, 64], non-causal, scale 1/8; and the uncached decoder,
// top-left causal). O = softmax(scale * Q K^T) V per (b, h), with an online softmax in the
// log2 domain.
//
// Three kernels share the arithmetic below:
//   * dense_fwd_kernel (non-causal; the encoder): 512-thread workgroups of eight 64-query
//     wavefronts (two per SIMD), K/V tiles of 64 keys in four LDS buffers, Q and O moved
//     through LDS as whole rows. Its own comment block gives the details.
//   * dense_mfma_kernel (causal): eight 32-query wavefronts per workgroup (~120 VGPRs, four
//     wavefronts per SIMD), three LDS buffers with V transposed at staging time, and the
//     causal diagonal handled per wavefront (keys past a wavefront's last query are skipped).
//   * dense_split_kernel (non-causal, grids smaller than the chip): the same tile staging, with
//     each query group's keys split over two wavefronts that merge at the end (256-query
//     blocks); dense_split4_kernel splits each group's keys over four wavefronts (128-query
//     blocks, 128-key tiles).
// Each 64-key tile is consumed as two 32-key sub-steps.
//
// Transposed products. A wavefront computes S^T = K Q^T with v_mfma_f32_32x32x16 (A = K from
// LDS, B = Q kept in registers), so a lane owns whole query COLUMNS of S: the row max and row
// sum are in-lane work plus one exchange between the two 32-lane halves, and the output rescale
// is per lane. The output is produced transposed too, O^T = V^T P^T (A = V^T from LDS, B = P
// straight from the S accumulators). For P to serve as the B operand without shuffles, the K
// rows feeding S^T are loaded in a permuted order so that accumulator a of lane l holds key
// 16*(a>>3) + 8*(l>>5) + (a&7) of its 32-key block: accumulators 8c..8c+7 are then the eight
// consecutive keys the lane supplies for 16-key chunk c of the PV product.
//
// VALU diet (at head_dim 64 the softmax VALU work rivals the MFMA work, and on gfx950 the two
// largely serialise):
//   * Q is pre-scaled by scale*log2(e) once; fmax runs without NaN canonicalisation (the file
//     is built with -fno-honor-nans; masked scores are -inf, never NaN).
//   * Lazy rescaling: the running max only moves when a score exceeds it by more than kTau
//     (causal kernel: checked against the step's max) or when a step's row sum exceeds
//     kSumLimit (non-causal kernel: the sum is needed anyway, the max is not); P values up to
//     2^8 / 2^10 are exact enough in bf16 and harmless in fp32 sums, and in steady state the
//     output accumulator is never rescaled.
//   * Row sums are plain fp32 adds of the unrounded P into four independent partial sums.
//     (v_dot2 of the packed P against (1, 1) issues half as many instructions, but measured on
//     gfx950 it costs 1.6x an add and overlaps the other wavefront's MFMAs far less: 23% vs
//     ~60%; the adds are 2.5% faster overall.)
//
// Grid. One workgroup per (b, h, query block), flattened and remapped so that the query blocks
// of one (b, h) land on the same XCD (work-group ids are dealt round-robin over the 8 XCDs):
// they then share K/V through that XCD's L2.
#include "kv_dup.h"
#include "wdrz_common.h"
#include "wdrz_launch.h"
#include "dense_loop.inc"

#include <type_traits>

namespace wdrz {

namespace {

constexpr int kBN = 64;               // key rows per LDS tile
constexpr int kBS = 32;               // key rows per sub-step
constexpr int kPitchK = kHeadDim + 8; // K tile row pitch in elements (16-byte pad)
constexpr int kNumBuf = 3;            // LDS tile buffers
constexpr int kNumCus = 256;          // compute units of an MI355X
constexpr float kTau = 8.0f;          // lazy-rescale threshold (log2 units), causal kernel
constexpr float kSumLimit = 1024.0f;  // per-step row-sum limit of the non-causal kernel

template <typename T> struct Mfma;
template <> struct Mfma<Bf16> {
  typedef bf16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
  static __device__ __forceinline__ float widen_lo(uint32_t w) { return bf16_lo(w); }
  static __device__ __forceinline__ float widen_hi(uint32_t w) { return bf16_hi(w); }
};
template <> struct Mfma<F16> {
  typedef f16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
  static __device__ __forceinline__ float widen_lo(uint32_t w) { return f16_lo(w); }
  static __device__ __forceinline__ float widen_hi(uint32_t w) { return f16_hi(w); }
};


// max of x over the two 32-lane halves of the wavefront (every lane gets the result)
__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// V^T tile: 64 rows (head dims) x 64 keys, 128-byte rows, 16-byte key chunks XOR-swizzled by
// the row so that both the transposing dword stores and the 16-byte operand reads (16
// consecutive rows per pass) spread over all banks.
__device__ __forceinline__ int vt_index(int d, int key) {
  const int f = ((d >> 1) ^ (d >> 4)) & 7;
  return d * kBN + ((((key >> 3) ^ f) & 7) << 3) + (key & 7);
}

// Wave issue priority around MFMA sections: while this wavefront feeds the matrix core, the
// SIMD's arbiter prefers it over wavefronts running softmax VALU work, so the matrix pipe is
// not left idle between MFMAs (measured on gfx950 with two wavefronts per SIMD: +15% for the
// encoder shape).
template <int P>
__device__ __forceinline__ void mfma_priority() {
  __builtin_amdgcn_s_setprio(P);
}

// QB: 32-query blocks per wavefront; NW: wavefronts per workgroup.
template <typename T, bool CAUSAL, int QB, int NW>
__global__ __launch_bounds__(NW * 64) void dense_mfma_kernel(DenseArgs a) {
  constexpr int kThreads = NW * 64;
  constexpr int kBM = 32 * QB * NW;  // query rows per workgroup
  typedef typename Mfma<T>::op_t op_t;
  typedef uint16_t e_t;
  __shared__ __attribute__((aligned(16))) e_t sK[kNumBuf][kBN * kPitchK];
  __shared__ __attribute__((aligned(16))) e_t sVt[kNumBuf][kHeadDim * kBN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hl = lane >> 5;  // lane half
  const int l32 = lane & 31;

  const int n_qblk = (a.Lq + kBM - 1) / kBM;
  int qblk, bh;
  if (CAUSAL) {
    // Heaviest blocks first: under the top-left mask the last query block of a head needs the
    // most keys, so all (b, h)'s last blocks are dispatched before their earlier ones and the
    // light blocks fill the slots the heavy ones leave (448 x 448 at B=16: 35 -> 32.5 us).
    const int n_bh = a.B * a.H;
    qblk = n_qblk - 1 - (int)blockIdx.x / n_bh;
    bh = (int)blockIdx.x % n_bh;
  } else {
    const int tile_id = remap_xcd(blockIdx.x, gridDim.x);
    qblk = tile_id % n_qblk;
    bh = tile_id / n_qblk;
  }
  const int b = bh / a.H, h = bh % a.H;

  const e_t* Q = reinterpret_cast<const e_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const e_t* K = reinterpret_cast<const e_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const e_t* V = reinterpret_cast<const e_t*>(a.v) + b * a.vs[0] + h * a.vs[1];
  e_t* O = reinterpret_cast<e_t*>(a.o) + b * a.os[0] + h * a.os[1];

  const int q_wg = qblk * kBM;
  // Causal: the two wavefronts that share a SIMD (w and w + 4) take query blocks s and 7 - s, so
  // every SIMD gets the same number of key steps under the mask (1 + 8, 2 + 7, ...)
  const int wblk = (CAUSAL && NW == 8) ? (wave < 4 ? wave : 11 - wave) : wave;
  const int q_wave = q_wg + wblk * 32 * QB;
  const float c = a.c;

  // Q operand (B of S^T = K Q^T), pre-scaled by c: lane holds query q_wave + qb*32 + l32,
  // dims ks*16 + hl*8 + 0..7.
  op_t qreg[QB][4];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qi = min(q_wave + qb * 32 + l32, a.Lq - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4 raw = load16(Q + qi * a.qs[2] + ks * 16 + hl * 8);
      u32x4 sc;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sc[e] = Mfma<T>::pack(Mfma<T>::widen_lo(raw[e]) * c, Mfma<T>::widen_hi(raw[e]) * c);
      // Opaque to the optimiser: keeps the scaled Q resident instead of being recomputed
      // from the raw load in every sub-step.
      asm volatile("" : "+v"(sc));
      qreg[qb][ks] = __builtin_bit_cast(op_t, sc);
    }
  }

  // Keys needed by the workgroup and by this wavefront.
  int k_lim = a.Lk;
  if (CAUSAL) k_lim = min(a.Lk, q_wg + kBM);
  const int n_tiles = (k_lim + kBN - 1) / kBN;
  const int n_sub = (k_lim + kBS - 1) / kBS;
  int n_sub_w = n_sub;  // sub-steps this wavefront computes (causal: fewer for early rows)
  if (CAUSAL) n_sub_w = min(n_sub, (min(a.Lk, q_wave + 32 * QB) + kBS - 1) / kBS);

  // Tile staging. K: 64 rows x 128 B, each 16-byte piece loaded and stored as is.
  // V: transposed into V^T; a thread owns a key pair and a run of dims, packing the pair's
  // values of one dim into one dword store.
  constexpr int kKPerThr = (kBN * kHeadDim / 8) / kThreads;  // 16-byte K pieces per thread
  constexpr int kVDims = (kBN / 2) * kHeadDim / kThreads;     // dims per thread per key pair
  static_assert(kKPerThr >= 1 && (kVDims == 8 || kVDims == 4), "tile staging shape");
  typedef typename std::conditional<kVDims == 8, u32x4, u32x2>::type vpiece_t;
  u32x4 pk[kKPerThr];
  vpiece_t pv[2];
  const int vkp = tid / (kHeadDim / kVDims);        // key pair
  const int vd0 = (tid % (kHeadDim / kVDims)) * kVDims;
  auto gload = [&](int kt, u32x4 (&gk)[kKPerThr], vpiece_t (&gv)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < kKPerThr; ++r) {
      const int piece = tid + r * kThreads;
      const int key = min(kt * kBN + (piece >> 3), a.Lk - 1);
      gk[r] = load16(K + key * a.ks[2] + (piece & 7) * 8);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = min(kt * kBN + 2 * vkp + i, a.Lk - 1);
      gv[i] = *reinterpret_cast<const vpiece_t*>(V + key * a.vs[2] + vd0);
    }
  };
  auto lstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < kKPerThr; ++r) {
      const int piece = tid + r * kThreads;
      *reinterpret_cast<u32x4*>(&sK[buf][(piece >> 3) * kPitchK + (piece & 7) * 8]) = pk[r];
    }
#pragma unroll
    for (int e = 0; e < kVDims / 2; ++e) {
      const uint32_t lo0 = pv[0][e] & 0xffffu, hi0 = pv[0][e] >> 16;
      const uint32_t lo1 = pv[1][e] & 0xffffu, hi1 = pv[1][e] >> 16;
      *reinterpret_cast<uint32_t*>(&sVt[buf][vt_index(vd0 + 2 * e, 2 * vkp)]) = lo0 | (lo1 << 16);
      *reinterpret_cast<uint32_t*>(&sVt[buf][vt_index(vd0 + 2 * e + 1, 2 * vkp)]) = hi0 | (hi1 << 16);
    }
  };

  // Permuted key row this lane feeds as the A operand of S^T.
  const int pm = l32;
  const int pi_row = 16 * ((pm >> 3) >> 1) + 8 * ((pm >> 2) & 1) + 4 * ((pm >> 3) & 1) + (pm & 3);

  f32x16 acc_o[2][QB];  // [db][qb]: O^T rows d = db*32 + ..., column = query
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < QB; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc_o[i][j][x] = 0.f;
  float m_run[QB], l_part[QB][4];  // running max (scaled log2 units); 4 partial row sums
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) l_part[qb][j] = 0.f;
  }
  op_t pprev[QB][2];  // [qb][chunk] P of the previous sub-step

  gload(0, pk, pv);
  lstore(0);
  __syncthreads();

  for (int s = 0; s <= n_sub; ++s) {
    const int t = s >> 1;  // tile of this sub-step
    const int kb = s & 1;  // 32-key half of the tile
    const int buf = t % kNumBuf;
    if (kb == 0 && t + 1 < n_tiles) gload(t + 1, pk, pv);

    const bool do_s = s < n_sub_w;
    const bool do_pv = s >= 1 && s - 1 < n_sub_w;
    f32x16 sacc[QB];
    mfma_priority<1>();
    if (do_s) {
      // ---- S^T = K (cQ)^T ----
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const op_t ka = __builtin_bit_cast(
            op_t, *reinterpret_cast<const u32x4*>(&sK[buf][(kb * 32 + pi_row) * kPitchK + ks * 16 + hl * 8]));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[qb] = Mfma<T>::run(ka, qreg[qb][ks], ks == 0 ? f32x16{} : sacc[qb]);
      }
    }
    if (do_pv) {
      // ---- O^T += V^T P_{s-1}^T ----
      const int sp = s - 1;
      const int bufp = (sp >> 1) % kNumBuf;
      const int kbp = sp & 1;
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const op_t va = __builtin_bit_cast(
              op_t, *reinterpret_cast<const u32x4*>(&sVt[bufp][vt_index(db * 32 + l32, kbp * 32 + ch * 16 + hl * 8)]));
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) acc_o[db][qb] = Mfma<T>::run(va, pprev[qb][ch], acc_o[db][qb]);
        }
      }
    }
    mfma_priority<0>();
    if (do_s) {
      // ---- mask (tail keys, causal diagonal) ----
      const int k0 = s * kBS;
      const bool need_mask = (k0 + kBS > a.Lk) || (CAUSAL && k0 + kBS - 1 > q_wave);
      if (need_mask) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const int qi = q_wave + qb * 32 + l32;
#pragma unroll
          for (int x = 0; x < 16; ++x) {
            const int key = k0 + 16 * (x >> 3) + 8 * hl + (x & 7);
            bool ok = key < a.Lk;
            if (CAUSAL) ok = ok && key <= qi;
            if (!ok) sacc[qb][x] = -INFINITY;
          }
        }
      }
      // ---- online softmax per query column ----
      float mx[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        // tree max over the lane's 16 scores, then across the two lane halves
        float m4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          m4[j] = fmaxf(fmaxf(sacc[qb][4 * j], sacc[qb][4 * j + 1]), fmaxf(sacc[qb][4 * j + 2], sacc[qb][4 * j + 3]));
        mx[qb] = half_swap_max(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]))) - m_run[qb];
      }
      // First sub-step: adopt the true max. Later: move the max only when it grew by > kTau.
      bool any_big = s == 0;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) any_big = any_big || mx[qb] > kTau;
      if (__any(any_big)) {
        // Side effect: stops the compiler from if-converting this rare path into an
        // unconditional rescale of the output accumulator.
        asm volatile("" ::: "memory");
        const bool first = s == 0;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float delta = first ? mx[qb] : fmaxf(mx[qb], 0.f);
          m_run[qb] += delta;
          if (!first) {
            const float alpha = fast_exp2(-delta);
#pragma unroll
            for (int j = 0; j < 4; ++j) l_part[qb][j] *= alpha;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
              for (int x = 0; x < 16; ++x) acc_o[db][qb][x] *= alpha;
          }
        }
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = fast_exp2(sacc[qb][ch * 8 + 2 * e] - m_run[qb]);
            const float p1 = fast_exp2(sacc[qb][ch * 8 + 2 * e + 1] - m_run[qb]);
            w[e] = Mfma<T>::pack(p0, p1);
            l_part[qb][e] = l_part[qb][e] + p0 + p1;
          }
          pprev[qb][ch] = __builtin_bit_cast(op_t, w);
        }
      }
    }
    // Stage the prefetched tile t+1 after the second sub-step of tile t. Its buffer last held
    // tile t-2, whose final PV ran in sub-step 2t-2, before the previous barrier.
    if (kb == 1 && t + 1 < n_tiles) {
      lstore((t + 1) % kNumBuf);
      __syncthreads();
    }
  }

  // ---- normalise and store: lane holds a query column, 4 consecutive dims per (db, i) ----
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    float l_run = (l_part[qb][0] + l_part[qb][1]) + (l_part[qb][2] + l_part[qb][3]);
    const float lt = l_run + __shfl_xor(l_run, 32);
    const float inv = 1.f / lt;
    const int qi = q_wave + qb * 32 + l32;
    if (qi < a.Lq) {
      e_t* orow = O + qi * a.os[2];
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = db * 32 + i * 8 + hl * 4;
          u32x2 w;
          w[0] = Mfma<T>::pack(acc_o[db][qb][i * 4 + 0] * inv, acc_o[db][qb][i * 4 + 1] * inv);
          w[1] = Mfma<T>::pack(acc_o[db][qb][i * 4 + 2] * inv, acc_o[db][qb][i * 4 + 3] * inv);
          *reinterpret_cast<u32x2*>(orow + d) = w;
        }
    }
  }
}

// ============================================================================================
// Many-query cached attention (flash_attn_with_kvcache with sq >= kPrefillMinSq; reference
// src/whisperdrz/model.py:42-67). Self (HAS_NEW, a prompt's prefill): for batch row b, query t of the sq new rows sees keys
// [0, cs + t] of the row's cache after the append, cs = cache_seqlens[b] -- keys below cs from
// the cache slot, the others straight from k_new / v_new -- and the workgroup appends its own
// query rows' new keys and values to the cache. The step structure is the causal kernel's above
// (256 queries in eight 32-query wavefronts, K/V tiles of 64 keys through three LDS buffers, V
// transposed at staging), so each new row's keys are read ~sq/256 times instead of once per
// 16-query block. Cross (no new rows, the prompt's cross-attention): every query sees all Lk
// cache rows and nothing is appended. Rows with invalid metadata (slot outside the pool; self:
// cs < 0 or cs + sq past the cache) get NaN output and no append.
// ============================================================================================
template <typename T, bool HAS_NEW>
__global__ __launch_bounds__(512, 4) void kv_prefill_kernel(KvArgs a) {
  constexpr int NW = 8;
  constexpr int kThreads = NW * 64;
  constexpr int kBM = 32 * NW;
  typedef typename Mfma<T>::op_t op_t;
  typedef uint16_t e_t;
  __shared__ __attribute__((aligned(16))) e_t sK[kNumBuf][kBN * kPitchK];
  __shared__ __attribute__((aligned(16))) e_t sVt[kNumBuf][kHeadDim * kBN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  // heaviest query blocks (the last ones of a row) first, as in the causal kernel
  const int n_qblk = (a.sq + kBM - 1) / kBM;
  const int qblk = n_qblk - 1 - (int)blockIdx.x / a.B;
  const int b = (int)blockIdx.x % a.B;
  const int h = blockIdx.y;
  const int slot = a.bidx ? a.bidx[b] : b;
  // self: pre-append length; cross (no new rows): every cache row is a key
  const int cs = HAS_NEW ? a.seqlens[b] : a.Lk;
  const int sq = a.sq;
  const int q_wg = qblk * kBM;
  const int q_wave = q_wg + wave * 32;

  char* const Ob = a.o + (int64_t)b * a.os[0] + (int64_t)h * a.os[2];
  if (slot < 0 || slot >= a.n_slots || (HAS_NEW && (cs < 0 || cs + sq > a.Lk))) {
    const int t = q_wave + l32;
    if (t < sq) {
      e_t* orow = reinterpret_cast<e_t*>(Ob + (int64_t)t * a.os[1]);
      const e_t nan16 = __is_same(T, Bf16) ? (e_t)0x7fc0 : (e_t)0x7e00;
#pragma unroll
      for (int d = 32 * hl; d < 32 * hl + 32; ++d) orow[d] = nan16;
    }
    return;  // the whole workgroup: no barrier follows
  }

  // other rows appending to this slot (kv_dup.h): usually none
  const KvDup dup = HAS_NEW ? kv_dup_classify(a, b, slot, cs) : KvDup{b, false};
  if (HAS_NEW && dup.general) {
    // generic path: this workgroup's queries, then the new rows of its query block that it wins
    __shared__ float sm_q[NW][kHeadDim];
    const int nq = min(kBM, sq - q_wg);
    kv_generic_rows<T, NW>(a, b, h, slot, cs, q_wg, nq, 0, a.Lk, true, sm_q,
                           [&](int t, int d, float o, float m, float l) {
                             (void)m;
                             char* orow = Ob + (int64_t)(q_wg + t) * a.os[1];
                             if constexpr (__is_same(T, Bf16))
                               reinterpret_cast<__bf16*>(orow)[d] = (__bf16)(o / l);
                             else
                               reinterpret_cast<_Float16*>(orow)[d] = (_Float16)(o / l);
                           });
    for (int idx = tid; idx < nq * 2 * 8; idx += kThreads) {
      const int t = idx / 16, which = (idx / 8) & 1, piece = idx % 8;
      int cw = 0;
      if (kv_dup_winner(a, slot, cs + q_wg + t, cw) != b) continue;
      const char* src = which ? a.vn + (int64_t)b * a.vns[0] + (int64_t)(q_wg + t) * a.vns[1] + (int64_t)h * a.vns[2]
                              : a.kn + (int64_t)b * a.kns[0] + (int64_t)(q_wg + t) * a.kns[1] + (int64_t)h * a.kns[2];
      char* dst = which ? a.vc + (int64_t)slot * a.vcs[0] + (int64_t)(cs + q_wg + t) * a.vcs[1] + (int64_t)h * a.vcs[2]
                        : a.kc + (int64_t)slot * a.kcs[0] + (int64_t)(cs + q_wg + t) * a.kcs[1] + (int64_t)h * a.kcs[2];
      reinterpret_cast<u32x4*>(dst)[piece] = reinterpret_cast<const u32x4*>(src)[piece];
    }
    return;
  }
  const char* const Qb = a.q + (int64_t)b * a.qs[0] + (int64_t)h * a.qs[2];
  const char* const Kc = a.kc + (int64_t)slot * a.kcs[0] + (int64_t)h * a.kcs[2];
  const char* const Vc = a.vc + (int64_t)slot * a.vcs[0] + (int64_t)h * a.vcs[2];
  // the new rows: those of the last row appending this same region (this row when alone)
  const char* const Kn = HAS_NEW ? a.kn + (int64_t)dup.src * a.kns[0] + (int64_t)h * a.kns[2] : nullptr;
  const char* const Vn = HAS_NEW ? a.vn + (int64_t)dup.src * a.vns[0] + (int64_t)h * a.vns[2] : nullptr;
  char* const Kw = a.kc + (int64_t)slot * a.kcs[0] + (int64_t)h * a.kcs[2];
  char* const Vw = a.vc + (int64_t)slot * a.vcs[0] + (int64_t)h * a.vcs[2];
  const float c = a.c;

  op_t qreg[4];
  {
    const int t = min(q_wave + l32, sq - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4 raw = load16(Qb + (int64_t)t * a.qs[1] + (ks * 16 + hl * 8) * 2);
      u32x4 sc;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sc[e] = Mfma<T>::pack(Mfma<T>::widen_lo(raw[e]) * c, Mfma<T>::widen_hi(raw[e]) * c);
      asm volatile("" : "+v"(sc));
      qreg[ks] = __builtin_bit_cast(op_t, sc);
    }
  }

  // keys of this workgroup: self [0, cs + min(sq, q_wg + kBM)), of this wavefront up to its last
  // row; cross: all cs = Lk rows
  const int k_lim = HAS_NEW ? cs + min(sq, q_wg + kBM) : cs;
  const int n_tiles = (k_lim + kBN - 1) / kBN;
  const int n_sub = (k_lim + kBS - 1) / kBS;
  const int n_sub_w =
      q_wave >= sq ? 0 : HAS_NEW ? min(n_sub, (cs + min(sq, q_wave + 32) + kBS - 1) / kBS) : n_sub;
  // new rows this workgroup appends: keys [app0, app1) (none for cross)
  const int app0 = HAS_NEW && dup.src == b ? cs + q_wg : 0, app1 = HAS_NEW && dup.src == b ? cs + min(sq, q_wg + kBM) : 0;

  constexpr int kKPerThr = (kBN * kHeadDim / 8) / kThreads;
  constexpr int kVDims = (kBN / 2) * kHeadDim / kThreads;
  static_assert(kKPerThr == 1 && kVDims == 4, "tile staging shape");
  u32x4 pk;
  u32x2 pv[2];
  const int vkp = tid / (kHeadDim / kVDims);
  const int vd0 = (tid % (kHeadDim / kVDims)) * kVDims;
  auto krow = [&](int key) -> const char* {
    return !HAS_NEW || key < cs ? Kc + (int64_t)key * a.kcs[1] : Kn + (int64_t)(key - cs) * a.kns[1];
  };
  auto vrow = [&](int key) -> const char* {
    return !HAS_NEW || key < cs ? Vc + (int64_t)key * a.vcs[1] : Vn + (int64_t)(key - cs) * a.vns[1];
  };
  auto gload = [&](int kt) __attribute__((always_inline)) {
    pk = load16(krow(min(kt * kBN + (tid >> 3), k_lim - 1)) + (tid & 7) * 16);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      pv[i] = *reinterpret_cast<const u32x2*>(vrow(min(kt * kBN + 2 * vkp + i, k_lim - 1)) + vd0 * 2);
  };
  // tile kt into LDS buffer buf; the workgroup's own new rows also go to the cache
  auto lstore = [&](int buf, int kt) __attribute__((always_inline)) {
    if (HAS_NEW) {
      const int kkey = kt * kBN + (tid >> 3);
      if (kkey >= app0 && kkey < app1) *reinterpret_cast<u32x4*>(Kw + (int64_t)kkey * a.kcs[1] + (tid & 7) * 16) = pk;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int vkey = kt * kBN + 2 * vkp + i;
        if (vkey >= app0 && vkey < app1) *reinterpret_cast<u32x2*>(Vw + (int64_t)vkey * a.vcs[1] + vd0 * 2) = pv[i];
      }
    }
    *reinterpret_cast<u32x4*>(&sK[buf][(tid >> 3) * kPitchK + (tid & 7) * 8]) = pk;
#pragma unroll
    for (int e = 0; e < kVDims / 2; ++e) {
      const uint32_t lo0 = pv[0][e] & 0xffffu, hi0 = pv[0][e] >> 16;
      const uint32_t lo1 = pv[1][e] & 0xffffu, hi1 = pv[1][e] >> 16;
      *reinterpret_cast<uint32_t*>(&sVt[buf][vt_index(vd0 + 2 * e, 2 * vkp)]) = lo0 | (lo1 << 16);
      *reinterpret_cast<uint32_t*>(&sVt[buf][vt_index(vd0 + 2 * e + 1, 2 * vkp)]) = hi0 | (hi1 << 16);
    }
  };

  const int pm = l32;
  const int pi_row = 16 * ((pm >> 3) >> 1) + 8 * ((pm >> 2) & 1) + 4 * ((pm >> 3) & 1) + (pm & 3);

  f32x16 acc_o[2];
#pragma unroll
  for (int x = 0; x < 16; ++x) acc_o[0][x] = acc_o[1][x] = 0.f;
  float m_run = 0.f, l_part[4] = {0.f, 0.f, 0.f, 0.f};
  op_t pprev[2];
  const int qi = q_wave + l32;  // this lane's query row (past sq: a duplicate, never stored)

  gload(0);
  lstore(0, 0);
  __syncthreads();

  for (int s = 0; s <= n_sub; ++s) {
    const int t = s >> 1;
    const int kb = s & 1;
    const int buf = t % kNumBuf;
    if (kb == 0 && t + 1 < n_tiles) gload(t + 1);

    const bool do_s = s < n_sub_w;
    const bool do_pv = s >= 1 && s - 1 < n_sub_w;
    f32x16 sacc;
    mfma_priority<1>();
    if (do_s) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const op_t ka = __builtin_bit_cast(
            op_t, *reinterpret_cast<const u32x4*>(&sK[buf][(kb * 32 + pi_row) * kPitchK + ks * 16 + hl * 8]));
        sacc = Mfma<T>::run(ka, qreg[ks], ks == 0 ? f32x16{} : sacc);
      }
    }
    if (do_pv) {
      const int sp = s - 1;
      const int bufp = (sp >> 1) % kNumBuf;
      const int kbp = sp & 1;
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const op_t va = __builtin_bit_cast(
              op_t, *reinterpret_cast<const u32x4*>(&sVt[bufp][vt_index(db * 32 + l32, kbp * 32 + ch * 16 + hl * 8)]));
          acc_o[db] = Mfma<T>::run(va, pprev[ch], acc_o[db]);
        }
    }
    mfma_priority<0>();
    if (do_s) {
      // mask: keys past this row's causal limit cs + qi (self) and past the workgroup's keys
      const int k0 = s * kBS;
      if (HAS_NEW ? k0 + kBS - 1 > cs + q_wave : k0 + kBS > k_lim) {
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          const int key = k0 + 16 * (x >> 3) + 8 * hl + (x & 7);
          if ((HAS_NEW && key > cs + qi) || key >= k_lim) sacc[x] = -INFINITY;
        }
      }
      float m4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        m4[j] = fmaxf(fmaxf(sacc[4 * j], sacc[4 * j + 1]), fmaxf(sacc[4 * j + 2], sacc[4 * j + 3]));
      const float mx = half_swap_max(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]))) - m_run;
      if (__any(s == 0 || mx > kTau)) {
        asm volatile("" ::: "memory");
        const bool first = s == 0;
        const float delta = first ? mx : fmaxf(mx, 0.f);
        m_run += delta;
        if (!first) {
          const float alpha = fast_exp2(-delta);
#pragma unroll
          for (int j = 0; j < 4; ++j) l_part[j] *= alpha;
#pragma unroll
          for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int x = 0; x < 16; ++x) acc_o[db][x] *= alpha;
        }
      }
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = fast_exp2(sacc[ch * 8 + 2 * e] - m_run);
          const float p1 = fast_exp2(sacc[ch * 8 + 2 * e + 1] - m_run);
          w[e] = Mfma<T>::pack(p0, p1);
          l_part[e] = l_part[e] + p0 + p1;
        }
        pprev[ch] = __builtin_bit_cast(op_t, w);
      }
    }
    if (kb == 1 && t + 1 < n_tiles) {
      lstore((t + 1) % kNumBuf, t + 1);
      __syncthreads();
    }
  }

  const float l_run = (l_part[0] + l_part[1]) + (l_part[2] + l_part[3]);
  const float inv = 1.f / (l_run + __shfl_xor(l_run, 32));
  if (qi < sq) {
    e_t* orow = reinterpret_cast<e_t*>(Ob + (int64_t)qi * a.os[1]);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = db * 32 + i * 8 + hl * 4;
        u32x2 w;
        w[0] = Mfma<T>::pack(acc_o[db][i * 4 + 0] * inv, acc_o[db][i * 4 + 1] * inv);
        w[1] = Mfma<T>::pack(acc_o[db][i * 4 + 2] * inv, acc_o[db][i * 4 + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + d) = w;
      }
  }
}

// Transposing LDS read (gfx950 ds_read_b64_tr_b16). Within each 16-lane group, lane i gets
// element (i % 4) of the 8-byte chunks read by lanes 4c + i/4 (c = 0..3) of its group: with
// every lane pointing at 4 consecutive dims of one key row, this turns a row-major
// [key][dim] tile into the dim-major operand an MFMA A-input needs.
// `p` must point into __shared__ memory: its low 32 bits are then the LDS byte offset.
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
#if __HIP_DEVICE_COMPILE__
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uint32_t)(uintptr_t)p);
  return __builtin_bit_cast(u32x2, v);
#else
  (void)p;
  return u32x2{0, 0};
#endif
}

// ============================================================================================
// Non-causal kernel (the encoder shape): 512-thread workgroups, eight wavefronts of 64 queries
// each (two per SIMD), one workgroup per (b, h, 512-query block).
//
// Per step s a wavefront issues PV(s-1) and S(s) (16 MFMAs at raised wave priority), reads the
// next step's K and V^T operands from LDS, then runs the softmax of S(s). On gfx950 the softmax
// VALU work and the MFMAs of the wavefronts sharing a SIMD largely serialise (a softmax waits
// for the score MFMAs issued just before it, queued in the matrix pipe behind the other
// wavefront's), so the step time is close to their sum: the VALU side is cut to 32 exp2,
// 16 packs, 32 adds (the row sums, which double as the rescale check) and one compare per
// step, and the subtraction of the running max is folded into the S accumulation, which
// starts from -m_run (cinit) instead of zero.
//
// K/V tiles of 64 keys are staged through registers into four LDS buffers (tile t+2 loaded
// while tile t is consumed), with one workgroup barrier per tile; the wavefronts otherwise run
// free. Q and O move through LDS at the start and end, so that global memory sees whole
// 128-byte head rows (the operand layouts would otherwise scatter 16- and 8-byte pieces over
// 32 rows per instruction, which measured ~2.7 TB/s for these transfers).
// ============================================================================================
constexpr int kFWaves = 8;
constexpr int kFThreads = kFWaves * 64;
constexpr int kFBM = 64 * kFWaves;  // queries per workgroup
constexpr int kFBuf = 4;            // LDS tile buffers
// The Q and O staging areas ([512 rows][kPitchK]) alias the tile buffers.
static_assert(kFBM * kPitchK <= 2 * kFBuf * kBN * kPitchK, "Q/O staging must fit the tile buffers");

template <typename T>
__global__ __launch_bounds__(kFThreads, 1) void dense_fwd_kernel(DenseArgs a) {
  typedef typename Mfma<T>::op_t op_t;
  typedef uint16_t e_t;
  // K tiles then V tiles, each row-major [key][dim] with a 16-byte pad per row; at the start
  // and end the same memory holds Q and O as [query][dim] rows.
  __shared__ __attribute__((aligned(16))) e_t smem[2 * kFBuf * kBN * kPitchK];
  e_t* const sK = smem;
  e_t* const sV = smem + kFBuf * kBN * kPitchK;
  constexpr int kTileElems = kBN * kPitchK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  const int n_qblk = (a.Lq + kFBM - 1) / kFBM;
  const int tile_id = remap_xcd(blockIdx.x, gridDim.x);
  const int qblk = tile_id % n_qblk;
  const int bh = tile_id / n_qblk;  // heads [0, n / n_qblk): an offset here costs 3.5% (register allocation)
  const int b = bh / a.H, h = bh % a.H;

  const e_t* Q = reinterpret_cast<const e_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const e_t* K = reinterpret_cast<const e_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const e_t* V = reinterpret_cast<const e_t*>(a.v) + b * a.vs[0] + h * a.vs[1];
  e_t* O = reinterpret_cast<e_t*>(a.o) + b * a.os[0] + h * a.os[1];
  const int q_blk0 = qblk * kFBM;
  const int q_wave = q_blk0 + wave * 64;
  const float c = a.c;

  // Row-contiguous transfers: thread tid moves 16-byte chunk (tid & 7) of rows tid/8 + 64*i.
  const int crow = tid >> 3, cd0 = (tid & 7) * 8;

  // Tile staging: one 16-byte piece of K and one of V per thread and tile.
  const e_t* kg = K + (int64_t)crow * a.ks[2] + cd0;
  const e_t* vg = V + (int64_t)crow * a.vs[2] + cd0;
  const e_t* kg_last = K + (int64_t)(a.Lk - 1) * a.ks[2] + cd0;
  const e_t* vg_last = V + (int64_t)(a.Lk - 1) * a.vs[2] + cd0;
  const int64_t k_tile = (int64_t)kBN * a.ks[2], v_tile = (int64_t)kBN * a.vs[2];
  u32x4 pk, pv;
  auto gload = [&](int kt) __attribute__((always_inline)) {
    const bool in = kt * kBN + crow < a.Lk;
    pk = load16(in ? kg + kt * k_tile : kg_last);
    pv = load16(in ? vg + kt * v_tile : vg_last);
  };
  const int st_off = crow * kPitchK + cd0;
  auto lstore = [&](int buf) __attribute__((always_inline)) {
    *reinterpret_cast<u32x4*>(&sK[buf * kTileElems + st_off]) = pk;
    *reinterpret_cast<u32x4*>(&sV[buf * kTileElems + st_off]) = pv;
  };

  const int n_tiles = (a.Lk + kBN - 1) / kBN;
  const int n_sub = (a.Lk + kBS - 1) / kBS;

  // ---- Q: whole rows from global memory into LDS, then each wavefront's operand registers,
  // pre-scaled by c (kept opaque so the scaled values stay resident) ----
  op_t qreg[2][4];
  {
    u32x4 qc[kFBM / 64];
#pragma unroll
    for (int i = 0; i < kFBM / 64; ++i) qc[i] = load16(Q + min(q_blk0 + crow + 64 * i, a.Lq - 1) * a.qs[2] + cd0);
    gload(0);
#pragma unroll
    for (int i = 0; i < kFBM / 64; ++i) *reinterpret_cast<u32x4*>(&smem[(crow + 64 * i) * kPitchK + cd0]) = qc[i];
    __syncthreads();
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 raw =
            *reinterpret_cast<const u32x4*>(&smem[(wave * 64 + qb * 32 + l32) * kPitchK + ks * 16 + hl * 8]);
        u32x4 sc;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          sc[e] = Mfma<T>::pack(Mfma<T>::widen_lo(raw[e]) * c, Mfma<T>::widen_hi(raw[e]) * c);
        asm volatile("" : "+v"(sc));
        qreg[qb][ks] = __builtin_bit_cast(op_t, sc);
      }
    __syncthreads();
  }

  // Per-lane LDS offsets. K operand: permuted key row (see the header comment), dims
  // ks*16 + hl*8. V^T operand through the transposing read: this lane points at key row
  // 8*(g>>1) + (j>>2) (+4 for the second half) and dims 16*(g&1) + 4*(j&3) of a 32-dim block,
  // where g is its 16-lane group and j its index in the group.
  const int pm = l32;
  const int pi_row = 16 * ((pm >> 3) >> 1) + 8 * ((pm >> 2) & 1) + 4 * ((pm >> 3) & 1) + (pm & 3);
  const int k_off = pi_row * kPitchK + hl * 8;
  const int g16 = lane >> 4, j16 = lane & 15;
  const int v_off = (8 * (g16 >> 1) + (j16 >> 2)) * kPitchK + 16 * (g16 & 1) + 4 * (j16 & 3);

  op_t kop[4], vop[2][2];  // operands of the next MFMA step: kop[ks], vop[ch][db]
  auto read_k = [&](int s) __attribute__((always_inline)) {
    const e_t* kb = &sK[((s >> 1) % kFBuf) * kTileElems + (s & 1) * 32 * kPitchK + k_off];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kop[ks] = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(kb + ks * 16));
  };
  auto read_v = [&](int s) __attribute__((always_inline)) {
    const e_t* vb = &sV[((s >> 1) % kFBuf) * kTileElems + (s & 1) * 32 * kPitchK + v_off];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const e_t* p = vb + ch * 16 * kPitchK + db * 32;
        const u32x2 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 4 * kPitchK);
        vop[ch][db] = __builtin_bit_cast(op_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
      }
  };

  f32x16 acc_o[2][2];  // [db][qb]: O^T rows d = db*32 + ..., column = query
  f32x16 sacc[2];      // [qb] scores of the current step, relative to m_run
  f32x16 cinit[2];     // [qb] -m_run: the starting value of every S accumulation
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      cinit[i][x] = 0.f;
      acc_o[0][i][x] = 0.f;
      acc_o[1][i][x] = 0.f;
    }
  float m_run[2] = {0.f, 0.f};
  float l_run[2] = {0.f, 0.f};
  op_t pcur[2][2];  // [qb][16-key chunk] P of the last softmax

  // Online softmax of step s for query block qb (on sacc[qb], scores relative to m_run).
  // Fast path: exponentiate against the current max and keep the step's row sum. Each lane's
  // sum covers 16 scores, so a sum above kSumLimit = 1024 means some score exceeded the max by
  // more than log2(1024/16) = 6 (or overflowed): only then is the true max taken, the state
  // rescaled and the step redone. P therefore stays below 1024, which bf16 P and the fp32
  // accumulators take exactly as well as P <= 1. The first step always takes the true max.
  // (This replaces a per-step max over the 16 scores: ~10 fewer VALU instructions per block.)
  auto exp_sum = [&](int qb) __attribute__((always_inline)) {
    float t[4];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p0 = fast_exp2(sacc[qb][ch * 8 + 2 * e]);
        const float p1 = fast_exp2(sacc[qb][ch * 8 + 2 * e + 1]);
        w[e] = Mfma<T>::pack(p0, p1);
        t[e] = ch == 0 ? p0 + p1 : t[e] + p0 + p1;
      }
      pcur[qb][ch] = __builtin_bit_cast(op_t, w);
    }
    return (t[0] + t[1]) + (t[2] + t[3]);
  };
  auto softmax = [&](int qb, int s) __attribute__((always_inline)) {
    const int k0 = s * kBS;
    if (k0 + kBS > a.Lk) {
#pragma unroll
      for (int x = 0; x < 16; ++x)
        if (k0 + 16 * (x >> 3) + 8 * hl + (x & 7) >= a.Lk) sacc[qb][x] = -INFINITY;
    }
    float st = s == 0 ? INFINITY : exp_sum(qb);
    if (__any(!(st <= kSumLimit))) {
      asm volatile("" ::: "memory");  // keep this rare path a branch
      // a tree of 3-input maxima (depth 3, not a chain of 8), then across the lane halves
      const f32x16& v = sacc[qb];
      const float t0 = fmaxf(fmaxf(v[0], v[1]), v[2]), t1 = fmaxf(fmaxf(v[3], v[4]), v[5]);
      const float t2 = fmaxf(fmaxf(v[6], v[7]), v[8]), t3 = fmaxf(fmaxf(v[9], v[10]), v[11]);
      const float t4 = fmaxf(fmaxf(v[12], v[13]), v[14]);
      const float mx = half_swap_max(fmaxf(fmaxf(fmaxf(t0, t1), t2), fmaxf(fmaxf(t3, t4), v[15])));
      const float delta = s == 0 ? mx : fmaxf(mx, 0.f);
      m_run[qb] += delta;
      if (s != 0) {
        const float alpha = fast_exp2(-delta);
        l_run[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int x = 0; x < 16; ++x) acc_o[db][qb][x] *= alpha;
      }
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        sacc[qb][x] -= delta;
        cinit[qb][x] = -m_run[qb];
      }
      st = exp_sum(qb);
    }
    l_run[qb] += st;
  };
  auto mfma_s = [&](int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) sacc[qb] = Mfma<T>::run(kop[ks], qreg[qb][ks], ks == 0 ? cinit[qb] : sacc[qb]);
  };
  auto mfma_pv = [&](int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int db = 0; db < 2; ++db) acc_o[db][qb] = Mfma<T>::run(vop[ch][db], pcur[qb][ch], acc_o[db][qb]);
  };

  // ---- first tiles (tile 0's loads were issued with Q) ----
  lstore(0);
  if (n_tiles > 1) {
    gload(1);
    lstore(1);
  }
  __syncthreads();
  read_k(0);

  // Step s, software-pipelined over the two query blocks so that each softmax has MFMAs of the
  // same wavefront to run under: [S(s) of block 0, PV(s-1) of block 1] [softmax(s) of block 0]
  // [S(s) of block 1, PV(s) of block 0] [softmax(s) of block 1]. Block 1's PV therefore lags
  // one step and runs on the V operands of step s-1, which are replaced only after it.
  for (int s = 0; s <= n_sub; ++s) {
    const int t = s >> 1;
    if (!(s & 1) && t + 2 < n_tiles) gload(t + 2);
    const bool has_s = s < n_sub;
    mfma_priority<1>();
    if (has_s) mfma_s(0);
    if (s >= 1) mfma_pv(1);
    mfma_priority<0>();
    __builtin_amdgcn_sched_barrier(0);
    if (has_s) read_v(s);
    if (has_s) softmax(0, s);
    __builtin_amdgcn_sched_barrier(0);
    mfma_priority<1>();
    if (has_s) {
      mfma_s(1);
      mfma_pv(0);
    }
    mfma_priority<0>();
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < n_sub) read_k(s + 1);
    if (has_s) softmax(1, s);
    // Tile t+2 replaces tile t-2, whose last reads (V of step 2t-3) came before the previous
    // tile's barrier; its first reads (K of step 2t+4, read in step 2t+3) come after this one.
    if (s & 1) {
      if (t + 2 < n_tiles) lstore((t + 2) % kFBuf);
      __syncthreads();
    }
  }
  if (!(n_sub & 1)) __syncthreads();  // the loop's last step (s = n_sub, even) had no barrier

  // ---- normalise, stage O^T through LDS as [query][dim] rows, store whole rows ----
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float inv = 1.f / (l_run[qb] + __shfl_xor(l_run[qb], 32));
    e_t* orow = &smem[(wave * 64 + qb * 32 + l32) * kPitchK];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x2 w;
        w[0] = Mfma<T>::pack(acc_o[db][qb][i * 4 + 0] * inv, acc_o[db][qb][i * 4 + 1] * inv);
        w[1] = Mfma<T>::pack(acc_o[db][qb][i * 4 + 2] * inv, acc_o[db][qb][i * 4 + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + db * 32 + i * 8 + hl * 4) = w;
      }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kFBM / 64; ++i) {
    const int qi = q_blk0 + crow + 64 * i;
    if (qi < a.Lq)
      store16(O + qi * a.os[2] + cd0, *reinterpret_cast<const u32x4*>(&smem[(crow + 64 * i) * kPitchK + cd0]));
  }
}

// ============================================================================================
// Non-causal kernel with a hand-scheduled main loop (the encoder shape): persistent, one
// 256-thread workgroup per CU, one wavefront per SIMD; an item is (b, h, query block) of 384
// queries (three 32-query blocks per wavefront) or 256 (two). With two wavefronts per SIMD
// (dense_fwd_kernel above) the softmax VALU work and the MFMAs of the two largely serialise; here
// a single instruction stream per SIMD interleaves them explicitly: while the VALU runs block b's
// softmax the matrix pipe runs the MFMAs of the block before it, whose inputs are all a phase old
// (gen_dense_loop.py, which emits the loop, gives the schedule and the register map). 384-query
// items also make the encoder launch whole rounds (B=16: 320 heads x 4 blocks = 5 x 256 items).
//
// The C++ around the loop turns the item's Q rows (in LDS, requested by the previous item's loop)
// into operand registers pre-scaled by scale*log2(e) and stores the first two K/V tiles into LDS
// (the loop requests the next ones itself, straight into LDS); the loop code also runs the last
// (partial) steps, and the C++ normalises and stores O through LDS as whole rows.
// ============================================================================================
constexpr int kPWaves = 4;
constexpr int kPThreads = kPWaves * 64;
constexpr int kPTile = kBN * 64;  // elements of one 64-key tile buffer (unpadded 128-byte rows, swizzled)
constexpr int kPMinKeys = 64;     // the loop needs two tiles up front

typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// A raw buffer resource over [base, base + bytes): loads past the end return zero.
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)(uintptr_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32) & 0xffff);  // stride 0
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;  // 32-bit data format, no swizzle
  return r;
}

// The same resource for the buffer load / store builtins (stores past the end are dropped).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_res(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Registers the generated loop uses beyond its operands (gen_dense_loop.py has the map).
#define WDRZ_PIPE_CLOBBERS \
  "v0", "v1", "v2", "v3", "v4", "v5", "v6", "v7", "v8", "v9", "v10", "v11", "v12", "v13", "v14", "v15", \
  "v16", "v17", "v18", "v19", "v20", "v21", "v22", "v23", "v24", "v25", "v26", "v27", "v28", "v29", "v30", \
  "v31", "v32", "v33", "v34", "v35", "v36", "v37", "v38", "v39", "v40", "v41", "v42", "v43", "v44", "v45", \
  "v46", "v47", "v48", "v49", "v50", "v51", "v52", "v53", "v54", "v55", "v56", "v57", "v58", "v59", "v60", \
  "v61", "v62", "v63", "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", \
  "v76", "v77", "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87", "v88", "v89", "v90", \
  "v91", "v92", "v93", "v94", "v95", "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104", \
  "v105", "v106", "v107", "v108", "v109", "v110", "v111", "v112", "v113", "v114", "v115", "v116", "v117", \
  "v118", "v119", "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127", "v128", "v129", "v130", \
  "v131", "v132", "v133", "v134", "v135", "v148", "v149", "v150", "v151", "v152", "v153", "v154", "v159", \
  "v168", "v169", "v170", "v171", "v172", "v173", "v174", "v175", "v176", "v177", "v178", "v179", "v180", \
  "v181", "v182", "v183", "v184", "v185", "v186", "v187", "v188", "v189", "v190", "v191", "v192", "v193", \
  "v194", "v195", "v196", "v197", "v198", "v199", "v200", "v201", "v202", "v203", "v204", "v205", "v206", \
  "v207", "v208", "v209", "v210", "v211", "v212", "v213", "v214", "v215", "v225", "a144", "a145", "a146", \
  "a147", "a148", "a149", "a150", "a151", "a152", "a153", "a154", "a155", "a156", "a157", "a158", "a159", \
  "a160", "a161", "a162", "a163", "a164", "a165", "a166", "a167", "a168", "a169", "a170", "a171", "a172", \
  "a173", "a174", "a175", "a176", "a177", "a178", "a179", "a180", "a181", "a182", "a183", "a184", "a185", \
  "a186", "a187", "a188", "a189", "a190", "a191", "a192", "a193", "a194", "a195", "a196", "a197", "a198", \
  "a199", "a200", "a201", "a202", "a203", "a204", "a205", "a206", "a207", "s70", "s71", "s72", "s73", "s74", \
  "s75", "s76", "s77", "s78", "s79", "m0", "vcc", "scc", "memory"

// NB: 32-query blocks per wavefront (3: 384-query items; 2: 256-query items for query counts
// that 384 would pad by more than 15%, such as the DTW decoder's 448 and a prompt's 224).
template <typename T, int NB>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void dense_pipe_kernel(DenseArgs a) {
  typedef typename Mfma<T>::op_t op_t;
  typedef uint16_t e_t;
  static_assert(NB == 2 || NB == 3, "two or three blocks per wavefront");
  constexpr int kPBM = 32 * NB * kPWaves;   // queries per item
  constexpr int kPQElems = kPBM * 64;       // the Q area: kPBM rows of 64 elements
  constexpr int kPQPieces = kPBM * 128 / kPThreads / 16;  // 1 KB Q prefetch pieces per wavefront
  constexpr int kWQ = 32 * NB;              // queries per wavefront
  // [Q rows: kPBM x 128 B, 16-byte chunks XOR-swizzled by the row] [four K tile buffers] [four V
  // tile buffers] (tiles row-major [key][dim], 128-byte rows, chunks XOR-swizzled); O is staged
  // through the tile buffers at the end of each item
  __shared__ __attribute__((aligned(16))) e_t smem[kPQElems + 8 * kPTile];
  e_t* const tiles = smem + kPQElems;
  static_assert(kPBM * kPitchK <= 8 * kPTile, "O staging must fit the tile buffers");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hl = lane >> 5;
  const int l32 = lane & 31;
  const float c = a.c;
  const int n_qblk = (a.Lq + kPBM - 1) / kPBM;
  const int n_items = a.B * a.H * n_qblk;

  // Row-contiguous transfers: thread tid moves 16-byte chunk (tid & 7) of rows tid/8 + 32*i.
  const int crow = tid >> 3, cd0 = (tid & 7) * 8;
  const int rs_k = (int)a.ks[2] * 2, rs_v = (int)a.vs[2] * 2, rs_q = (int)a.qs[2] * 2;  // row strides, bytes

  // The per-item pointers: item id (dispatch order) -> (b, h, query block), XCD-aware.
  struct Item {
    const e_t *q, *k, *v;
    e_t* o;
    int q0;
    bool bad;  // the row's slot is outside the cache: NaN output
  };
  auto item_of = [&](int id) {
    const int t = remap_xcd(id, n_items);
    const int qblk = t % n_qblk, bh = t / n_qblk;
    const int b = bh / a.H, h = bh % a.H;
    const int sl = a.slot ? a.slot[b] : b;
    Item it;
    it.bad = a.slot && (sl < 0 || sl >= a.n_slots);
    const int bk = it.bad ? 0 : sl;
    it.q = reinterpret_cast<const e_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
    it.k = reinterpret_cast<const e_t*>(a.k) + bk * a.ks[0] + h * a.ks[1];
    it.v = reinterpret_cast<const e_t*>(a.v) + bk * a.vs[0] + h * a.vs[1];
    it.o = reinterpret_cast<e_t*>(a.o) + b * a.os[0] + h * a.os[1];
    it.q0 = qblk * kPBM;
    return it;
  };
  // Global transfers through buffer resources bounded by the tensor (32-bit offsets, no
  // per-row 64-bit address arithmetic; rows past the end load as zero, stores there are dropped)
  const uint32_t k_bytes = (uint32_t)((a.Lk - 1) * rs_k + 128), v_bytes = (uint32_t)((a.Lk - 1) * rs_v + 128);
  auto tile_load = [&](const Item& it, int kt, u32x4 (&st)[4]) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rk = buffer_res(it.k, k_bytes), rv = buffer_res(it.v, v_bytes);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t r = (uint32_t)(kt * kBN + crow + 32 * i);
      st[i] = buf_load16(rk, r * rs_k + cd0 * 2);
      st[2 + i] = buf_load16(rv, r * rs_v + cd0 * 2);
    }
  };
  // tile layout: chunk c (16 bytes) of row r at element 64 r + 8 (c ^ ((r >> 1) & 7)) (the
  // operand reads of 16 lanes then touch 16 distinct 16-byte bank groups)
  auto tile_store = [&](int buf, const u32x4 (&st)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = crow + 32 * i;
      const int off = row * 64 + (((tid & 7) ^ ((row >> 1) & 7)) << 3);
      *reinterpret_cast<u32x4*>(&tiles[buf * kPTile + off]) = st[i];
      *reinterpret_cast<u32x4*>(&tiles[(4 + buf) * kPTile + off]) = st[2 + i];
    }
  };
  // Q rows through registers into the swizzled Q area (the first item; short keys)
  auto q_load_sync = [&](const Item& it) __attribute__((always_inline)) {
    u32x4 qc[kPBM / 32];
    const __amdgpu_buffer_rsrc_t rq =
        buffer_res(it.q + (int64_t)it.q0 * a.qs[2], (uint32_t)((min(kPBM, a.Lq - it.q0) - 1) * rs_q + 128));
#pragma unroll
    for (int i = 0; i < kPBM / 32; ++i) qc[i] = buf_load16(rq, (uint32_t)(crow + 32 * i) * rs_q + cd0 * 2);
#pragma unroll
    for (int i = 0; i < kPBM / 32; ++i) {
      const int row = crow + 32 * i;
      *reinterpret_cast<u32x4*>(&smem[row * 64 + (((tid & 7) ^ (row & 7)) << 3)]) = qc[i];
    }
  };

  // ---- constants of the generated loop ----
  const int n_sub = (a.Lk + kBS - 1) / kBS;
  const int n_iter = (a.Lk / kBS) / 2;
  const int n_rest = n_sub - 2 * n_iter;     // 0, 1 or 2
  const int rem = a.Lk - kBS * (n_sub - 1);  // valid keys of the last step
  // the next item's Q rows are requested by the loop code (one 1 KB piece per wavefront and
  // iteration) when the loop has the iterations for it
  const int n_pf = n_iter >= kPQPieces ? kPQPieces : 0;
  // LDS byte offsets of this lane's operand reads in the swizzled tiles: the permuted K rows,
  // one base per 16-key chunk ks; V^T through the transposing read, one base per 32-dim half db
  // and 4-row offset s (their chunk positions differ)
  const int pm = l32;
  const int pi_row = 16 * ((pm >> 3) >> 1) + 8 * ((pm >> 2) & 1) + 4 * ((pm >> 3) & 1) + (pm & 3);
  const int g16 = lane >> 4, j16 = lane & 15;
  const uint32_t tbase = kPQElems * 2;  // byte offset of the tile buffers
  u32x4 kl;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) kl[ks] = tbase + pi_row * 128 + (((2 * ks + hl) ^ ((pi_row >> 1) & 7)) << 4);
  typedef uint32_t u32x8v __attribute__((ext_vector_type(8)));
  u32x8v vl;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int sr = 0; sr < 2; ++sr) {
      const int r = 8 * (g16 >> 1) + (j16 >> 2) + 4 * sr;
      const int cc = 2 * (g16 & 1) + ((j16 & 3) >> 1) + 4 * db;
      vl[2 * db + sr] = tbase + r * 128 + ((cc ^ ((r >> 1) & 7)) << 4) + 8 * (j16 & 1);
    }
  const uint32_t hl8 = 8 * hl;  // key offset of this lane half (masking)
  // the loop's LDS DMA: wavefront w requests rows 16 w .. 16 w + 15 of each K and V tile in two
  // 8-row pieces, lane l writing position l % 8 of row l / 8 of a piece and so fetching the
  // global chunk the swizzle puts there
  const int dmab = __builtin_amdgcn_readfirstlane(tbase + wave * 16 * 128);
  const uint32_t swz0 = (uint32_t)(((lane & 7) ^ (lane >> 4)) << 4);        // rows 16 w + l / 8
  const uint32_t swz1 = (uint32_t)(((lane & 7) ^ (4 + (lane >> 4))) << 4);  // rows 16 w + 8 + l / 8
  const int tsk = kBN * rs_k, tsv = kBN * rs_v;
  // the Q prefetch: this lane's piece of row 8j + lane/8 of its wavefront's rows, swizzled chunk
  const uint32_t qvoff = (uint32_t)((wave * kWQ + (lane >> 3)) * rs_q + (((lane & 7) ^ (lane >> 3)) << 4));
  const int qlds = __builtin_amdgcn_readfirstlane(wave * kWQ * 128), qstep = 8 * rs_q;

  // Persistent: each workgroup takes items id, id + G, ... (G = grid size, a multiple of 8 so an
  // item stays on its XCD). While item k runs, item k+1's Q rows arrive in the Q area; its first
  // two K/V tiles are requested before item k's output is written.
  int id = blockIdx.x;
  Item cur = item_of(id);
  u32x4 t0[4], t1[4];
  q_load_sync(cur);
  tile_load(cur, 0, t0);
  tile_load(cur, 1, t1);
  for (;;) {
    const int next_id = id + (int)gridDim.x;
    const bool has_next = next_id < n_items;
    const Item nxt = item_of(has_next ? next_id : id);
    __syncthreads();  // the Q rows are in place; the previous item is done with the tile buffers
    u32x16 q0, q1, q2 = u32x16{};
#pragma unroll
    for (int qb = 0; qb < NB; ++qb)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int row = wave * kWQ + qb * 32 + l32;
        const u32x4 raw = *reinterpret_cast<const u32x4*>(&smem[row * 64 + (((2 * ks + hl) ^ (row & 7)) << 3)]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t w = Mfma<T>::pack(Mfma<T>::widen_lo(raw[e]) * c, Mfma<T>::widen_hi(raw[e]) * c);
          (qb == 0 ? q0 : qb == 1 ? q1 : q2)[ks * 4 + e] = w;
        }
      }
    tile_store(0, t0);
    tile_store(1, t1);
    __syncthreads();  // tiles 0, 1 in place; every wavefront has its Q operands (the Q area is free)

    // ---- the generated loop and the remaining steps (the last one masked at Lk) ----
    const i32x4 srd_k = buffer_rsrc(cur.k, (uint32_t)((a.Lk - 1) * rs_k + 128));
    const i32x4 srd_v = buffer_rsrc(cur.v, (uint32_t)((a.Lk - 1) * rs_v + 128));
    const int nq_next = min(kPBM, a.Lq - nxt.q0);
    const i32x4 srd_q = buffer_rsrc(nxt.q + (int64_t)nxt.q0 * a.qs[2], (uint32_t)((nq_next - 1) * rs_q + 128));
    const int npf = has_next ? n_pf : 0;
    // global byte offsets of this lane's rows of tile 2 (the first the loop code requests)
    u32x4 voff;
    voff[0] = (2 * kBN + wave * 16 + (lane >> 3)) * rs_k + swz0;
    voff[1] = (2 * kBN + wave * 16 + 8 + (lane >> 3)) * rs_k + swz1;
    voff[2] = (2 * kBN + wave * 16 + (lane >> 3)) * rs_v + swz0;
    voff[3] = (2 * kBN + wave * 16 + 8 + (lane >> 3)) * rs_v + swz1;
    f32x16 acc_o[3][2];
    typedef float f32x3 __attribute__((ext_vector_type(3)));
    f32x3 lr;  // this lane's half of each block's row sum
#define WDRZ_PIPE_OPERANDS                                                                                    \
  : "={a[0:15]}"(acc_o[0][0]), "={a[16:31]}"(acc_o[0][1]), "={a[32:47]}"(acc_o[1][0]), "={a[48:63]}"(acc_o[1][1]), \
    "={a[64:79]}"(acc_o[2][0]), "={a[80:95]}"(acc_o[2][1]), "={v[156:158]}"(lr), "+{v[164:167]}"(voff)             \
  : "{a[96:111]}"(q0), "{a[112:127]}"(q1), "{a[128:143]}"(q2), "{v[136:139]}"(kl), "{v[140:147]}"(vl),              \
    "{v163}"(hl8), "{v224}"(qvoff), "{s[80:83]}"(srd_k), "{s[84:87]}"(srd_v), "{s[88:91]}"(srd_q), [n] "s"(n_iter),  \
    [r] "s"(n_rest), [rem] "s"(rem), [tsk] "s"(tsk), [tsv] "s"(tsv), [npf] "s"(npf), [qlds] "s"(qlds),               \
    [qstep] "s"(qstep), [dmab] "s"(dmab)                                                                          \
  : WDRZ_PIPE_CLOBBERS
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (__is_same(T, Bf16) && NB == 3)
      asm volatile(WDRZ_DENSE_LOOP_BF16 WDRZ_PIPE_OPERANDS);
    else if constexpr (__is_same(T, Bf16))
      asm volatile(WDRZ_DENSE_LOOP_BF16_NB2 WDRZ_PIPE_OPERANDS);
    else if constexpr (NB == 3)
      asm volatile(WDRZ_DENSE_LOOP_F16 WDRZ_PIPE_OPERANDS);
    else
      asm volatile(WDRZ_DENSE_LOOP_F16_NB2 WDRZ_PIPE_OPERANDS);
    __builtin_amdgcn_sched_barrier(0);
#undef WDRZ_PIPE_OPERANDS

    // the next item's first tiles, in flight while this item's output is written
    if (has_next) {
      tile_load(nxt, 0, t0);
      tile_load(nxt, 1, t1);
    }
    // ---- normalise, stage O^T through the tile buffers as [query][dim] rows, store whole rows ----
    __syncthreads();  // every wavefront is done with the tiles
#pragma unroll
    for (int qb = 0; qb < NB; ++qb) {
      const float inv = cur.bad ? __uint_as_float(0x7fc00000u) : 1.f / (lr[qb] + __shfl_xor(lr[qb], 32));
      e_t* orow = &tiles[(wave * kWQ + qb * 32 + l32) * kPitchK];
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          u32x2 w;
          w[0] = Mfma<T>::pack(acc_o[qb][db][i * 4 + 0] * inv, acc_o[qb][db][i * 4 + 1] * inv);
          w[1] = Mfma<T>::pack(acc_o[qb][db][i * 4 + 2] * inv, acc_o[qb][db][i * 4 + 3] * inv);
          *reinterpret_cast<u32x2*>(orow + db * 32 + i * 8 + hl * 4) = w;
        }
    }
    __syncthreads();
    const int rs_o = (int)a.os[2] * 2;
    const __amdgpu_buffer_rsrc_t ro =
        buffer_res(cur.o + (int64_t)cur.q0 * a.os[2], (uint32_t)((min(kPBM, a.Lq - cur.q0) - 1) * rs_o + 128));
#pragma unroll
    for (int i = 0; i < kPBM / 32; ++i)
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int,
                             *reinterpret_cast<const u32x4*>(&tiles[(crow + 32 * i) * kPitchK + cd0])),
          ro, (uint32_t)(crow + 32 * i) * rs_o + cd0 * 2, 0, 0);
    if (!has_next) break;
    if (npf == 0) q_load_sync(nxt);  // (too few iterations to request it during the loop)
    id = next_id;
    cur = nxt;
  }
}

// ============================================================================================
// Key-split kernel (non-causal, small grids): a workgroup holds four query groups of 32*QB
// queries; each group is served by two wavefronts on the same SIMD (waves g and g+4), one per
// 32-key half of every 64-key tile, which merge their (m, l, O) through LDS at the end. Per query
// this is half the keys per wavefront of the other kernels, so a launch that would leave CUs idle
// or run a short last round (the DTW decoder's 448 x 1500 cross-attention, single-window
// encoder calls) gets two to four times as many workgroups of half the length.
// ============================================================================================
template <typename T, int QB>
__global__ __launch_bounds__(512) void dense_split_kernel(DenseArgs a) {
  constexpr int NW = 8, NG = 4;
  constexpr int kThreads = NW * 64;
  constexpr int kBM = 32 * QB * NG;  // query rows per workgroup
  typedef typename Mfma<T>::op_t op_t;
  typedef uint16_t e_t;
  __shared__ __attribute__((aligned(16))) e_t sK[kNumBuf][kBN * kPitchK];
  __shared__ __attribute__((aligned(16))) e_t sVt[kNumBuf][kHeadDim * kBN];
  constexpr int kPart = 32 * QB + 2 * QB;  // floats per lane of a partial: O (2 x QB x 16), m, l
  __shared__ float smerge[NG][kPart][64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave % NG;
  const int kh = wave / NG;  // 32-key half of each tile
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  const int n_qblk = (a.Lq + kBM - 1) / kBM;
  const int tile_id = remap_xcd(blockIdx.x, gridDim.x);
  const int qblk = tile_id % n_qblk;
  const int bh = a.bh0 + tile_id / n_qblk;
  const int b = bh / a.H, h = bh % a.H;

  const e_t* Q = reinterpret_cast<const e_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const e_t* K = reinterpret_cast<const e_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const e_t* V = reinterpret_cast<const e_t*>(a.v) + b * a.vs[0] + h * a.vs[1];
  e_t* O = reinterpret_cast<e_t*>(a.o) + b * a.os[0] + h * a.os[1];

  const int q_wave = qblk * kBM + grp * 32 * QB;
  const float c = a.c;

  op_t qreg[QB][4];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qi = min(q_wave + qb * 32 + l32, a.Lq - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4 raw = load16(Q + qi * a.qs[2] + ks * 16 + hl * 8);
      u32x4 sc;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sc[e] = Mfma<T>::pack(Mfma<T>::widen_lo(raw[e]) * c, Mfma<T>::widen_hi(raw[e]) * c);
      asm volatile("" : "+v"(sc));
      qreg[qb][ks] = __builtin_bit_cast(op_t, sc);
    }
  }

  const int n_tiles = (a.Lk + kBN - 1) / kBN;

  // Tile staging, as in dense_mfma_kernel with eight wavefronts.
  constexpr int kKPerThr = (kBN * kHeadDim / 8) / kThreads;
  constexpr int kVDims = (kBN / 2) * kHeadDim / kThreads;
  static_assert(kKPerThr == 1 && kVDims == 4, "tile staging shape");
  u32x4 pk;
  u32x2 pv[2];
  const int vkp = tid / (kHeadDim / kVDims);
  const int vd0 = (tid % (kHeadDim / kVDims)) * kVDims;
  auto gload = [&](int kt) __attribute__((always_inline)) {
    const int key = min(kt * kBN + (tid >> 3), a.Lk - 1);
    pk = load16(K + key * a.ks[2] + (tid & 7) * 8);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kv = min(kt * kBN + 2 * vkp + i, a.Lk - 1);
      pv[i] = *reinterpret_cast<const u32x2*>(V + kv * a.vs[2] + vd0);
    }
  };
  auto lstore = [&](int buf) __attribute__((always_inline)) {
    *reinterpret_cast<u32x4*>(&sK[buf][(tid >> 3) * kPitchK + (tid & 7) * 8]) = pk;
#pragma unroll
    for (int e = 0; e < kVDims / 2; ++e) {
      const uint32_t lo0 = pv[0][e] & 0xffffu, hi0 = pv[0][e] >> 16;
      const uint32_t lo1 = pv[1][e] & 0xffffu, hi1 = pv[1][e] >> 16;
      *reinterpret_cast<uint32_t*>(&sVt[buf][vt_index(vd0 + 2 * e, 2 * vkp)]) = lo0 | (lo1 << 16);
      *reinterpret_cast<uint32_t*>(&sVt[buf][vt_index(vd0 + 2 * e + 1, 2 * vkp)]) = hi0 | (hi1 << 16);
    }
  };

  const int pm = l32;
  const int pi_row = 16 * ((pm >> 3) >> 1) + 8 * ((pm >> 2) & 1) + 4 * ((pm >> 3) & 1) + (pm & 3);

  f32x16 acc_o[2][QB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < QB; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc_o[i][j][x] = 0.f;
  float m_run[QB], l_part[QB][4];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) l_part[qb][j] = 0.f;
  }
  op_t pprev[QB][2];
  bool seen = false;  // this wavefront has processed at least one key

  gload(0);
  lstore(0);
  __syncthreads();

  // Step t: S of this wavefront's half of tile t, PV of its half of tile t-1.
  for (int t = 0; t <= n_tiles; ++t) {
    const int buf = t % kNumBuf;
    if (t + 1 < n_tiles) gload(t + 1);
    const bool do_s = t < n_tiles && (2 * t + kh) * kBS < a.Lk;
    const bool do_pv = t >= 1 && (2 * (t - 1) + kh) * kBS < a.Lk;
    f32x16 sacc[QB];
    mfma_priority<1>();
    if (do_s) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const op_t ka = __builtin_bit_cast(
            op_t, *reinterpret_cast<const u32x4*>(&sK[buf][(kh * 32 + pi_row) * kPitchK + ks * 16 + hl * 8]));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[qb] = Mfma<T>::run(ka, qreg[qb][ks], ks == 0 ? f32x16{} : sacc[qb]);
      }
    }
    if (do_pv) {
      const int bufp = (t - 1) % kNumBuf;
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const op_t va = __builtin_bit_cast(
              op_t, *reinterpret_cast<const u32x4*>(&sVt[bufp][vt_index(db * 32 + l32, kh * 32 + ch * 16 + hl * 8)]));
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) acc_o[db][qb] = Mfma<T>::run(va, pprev[qb][ch], acc_o[db][qb]);
        }
      }
    }
    mfma_priority<0>();
    if (do_s) {
      const int k0 = (2 * t + kh) * kBS;
      if (k0 + kBS > a.Lk) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
          for (int x = 0; x < 16; ++x)
            if (k0 + 16 * (x >> 3) + 8 * hl + (x & 7) >= a.Lk) sacc[qb][x] = -INFINITY;
      }
      float mx[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float m4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          m4[j] = fmaxf(fmaxf(sacc[qb][4 * j], sacc[qb][4 * j + 1]), fmaxf(sacc[qb][4 * j + 2], sacc[qb][4 * j + 3]));
        mx[qb] = half_swap_max(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]))) - m_run[qb];
      }
      const bool first = !seen;
      bool any_big = first;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) any_big = any_big || mx[qb] > kTau;
      if (__any(any_big)) {
        asm volatile("" ::: "memory");
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float delta = first ? mx[qb] : fmaxf(mx[qb], 0.f);
          m_run[qb] += delta;
          if (!first) {
            const float alpha = fast_exp2(-delta);
#pragma unroll
            for (int j = 0; j < 4; ++j) l_part[qb][j] *= alpha;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
              for (int x = 0; x < 16; ++x) acc_o[db][qb][x] *= alpha;
          }
        }
      }
      seen = true;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = fast_exp2(sacc[qb][ch * 8 + 2 * e] - m_run[qb]);
            const float p1 = fast_exp2(sacc[qb][ch * 8 + 2 * e + 1] - m_run[qb]);
            w[e] = Mfma<T>::pack(p0, p1);
            l_part[qb][e] = l_part[qb][e] + p0 + p1;
          }
          pprev[qb][ch] = __builtin_bit_cast(op_t, w);
        }
      }
    }
    // Buffer (t+1)%3 last held tile t-2, read by S in step t-2 and PV in step t-1, both before
    // the previous barrier.
    if (t + 1 < n_tiles) {
      lstore((t + 1) % kNumBuf);
      __syncthreads();
    }
  }

  // ---- merge the two halves of each group, normalise, store ----
  float lsum[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) lsum[qb] = (l_part[qb][0] + l_part[qb][1]) + (l_part[qb][2] + l_part[qb][3]);
  if (kh == 1) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int x = 0; x < 16; ++x) smerge[grp][(qb * 2 + db) * 16 + x][lane] = acc_o[db][qb][x];
      smerge[grp][32 * QB + qb][lane] = seen ? m_run[qb] : -INFINITY;
      smerge[grp][33 * QB + qb][lane] = lsum[qb];
    }
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float m1 = smerge[grp][32 * QB + qb][lane];
    const float m = fmaxf(m_run[qb], m1);  // half 0 always sees key 0
    const float a0 = fast_exp2(m_run[qb] - m), a1 = fast_exp2(m1 - m);
    const float lq = lsum[qb] * a0 + smerge[grp][33 * QB + qb][lane] * a1;
    const float inv = 1.f / (lq + __shfl_xor(lq, 32));
    const int qi = q_wave + qb * 32 + l32;
    if (qi < a.Lq) {
      e_t* orow = O + qi * a.os[2];
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = db * 32 + i * 8 + hl * 4;
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int x = i * 4 + r;
            v[r] = (acc_o[db][qb][x] * a0 + smerge[grp][(qb * 2 + db) * 16 + x][lane] * a1) * inv;
          }
          u32x2 w;
          w[0] = Mfma<T>::pack(v[0], v[1]);
          w[1] = Mfma<T>::pack(v[2], v[3]);
          *reinterpret_cast<u32x2*>(orow + d) = w;
        }
    }
  }
}

// ============================================================================================
// Key-split kernel in quarters (the 128-query form of the above): each 32-query group is served
// by four wavefronts, one per 32-key quarter of every 128-key tile, so every SIMD interleaves four
// dependent score -> softmax -> PV chains instead of two (a single encoder window: 29-30 -> 26 us;
// the DTW cross-attention's key-split heads ~7% faster). 16 wavefronts, 128 queries per
// workgroup; the quarters' (m, l, O) merge through LDS that the tile buffers free after the loop.
// ============================================================================================
template <typename T>
__global__ __launch_bounds__(1024) void dense_split4_kernel(DenseArgs a) {
  constexpr int NG = 4, KS = 4, NW = NG * KS;
  constexpr int kThreads = NW * 64;
  constexpr int kBM = 32 * NG;        // queries per workgroup
  constexpr int kTB = 32 * KS;        // keys per tile
  constexpr int kPart = 34;           // floats per lane of a partial: O (2 x 16), m, l
  typedef typename Mfma<T>::op_t op_t;
  typedef uint16_t e_t;
  constexpr int kKBytes = kNumBuf * kTB * kPitchK * 2;
  constexpr int kVBytes = kNumBuf * 2 * kHeadDim * kBN * 2;
  constexpr int kMBytes = NG * (KS - 1) * kPart * 64 * 4;
  constexpr int kLds = kKBytes + kVBytes > kMBytes ? kKBytes + kVBytes : kMBytes;
  __shared__ __attribute__((aligned(16))) char lds[kLds];
  e_t (*sK)[kTB * kPitchK] = reinterpret_cast<e_t (*)[kTB * kPitchK]>(lds);
  e_t (*sVt)[2][kHeadDim * kBN] = reinterpret_cast<e_t (*)[2][kHeadDim * kBN]>(lds + kKBytes);
  float (*smerge)[KS - 1][kPart][64] = reinterpret_cast<float (*)[KS - 1][kPart][64]>(lds);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave % NG;
  const int kh = wave / NG;  // key quarter of each tile
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  const int n_qblk = (a.Lq + kBM - 1) / kBM;
  const int tile_id = remap_xcd(blockIdx.x, gridDim.x);
  const int qblk = tile_id % n_qblk;
  const int bh = a.bh0 + tile_id / n_qblk;
  const int b = bh / a.H, h = bh % a.H;

  const e_t* Q = reinterpret_cast<const e_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const e_t* K = reinterpret_cast<const e_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const e_t* V = reinterpret_cast<const e_t*>(a.v) + b * a.vs[0] + h * a.vs[1];
  e_t* O = reinterpret_cast<e_t*>(a.o) + b * a.os[0] + h * a.os[1];
  const int q_wave = qblk * kBM + grp * 32;
  const float c = a.c;

  op_t qreg[4];
  {
    const int qi = min(q_wave + l32, a.Lq - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4 raw = load16(Q + qi * a.qs[2] + ks * 16 + hl * 8);
      u32x4 sc;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sc[e] = Mfma<T>::pack(Mfma<T>::widen_lo(raw[e]) * c, Mfma<T>::widen_hi(raw[e]) * c);
      asm volatile("" : "+v"(sc));
      qreg[ks] = __builtin_bit_cast(op_t, sc);
    }
  }

  const int n_tiles = (a.Lk + kTB - 1) / kTB;
  u32x4 pk;
  u32x2 pv[2];
  const int vkp = tid >> 4;            // key pair 0..63 of the tile
  const int vd0 = (tid & 15) * 4;      // 4 dims
  auto gload = [&](int kt) __attribute__((always_inline)) {
    const int key = min(kt * kTB + (tid >> 3), a.Lk - 1);
    pk = load16(K + key * a.ks[2] + (tid & 7) * 8);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kv = min(kt * kTB + 2 * vkp + i, a.Lk - 1);
      pv[i] = *reinterpret_cast<const u32x2*>(V + kv * a.vs[2] + vd0);
    }
  };
  auto lstore = [&](int buf) __attribute__((always_inline)) {
    *reinterpret_cast<u32x4*>(&sK[buf][(tid >> 3) * kPitchK + (tid & 7) * 8]) = pk;
    const int sub = (2 * vkp) >> 6, kin = (2 * vkp) & 63;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t lo0 = pv[0][e] & 0xffffu, hi0 = pv[0][e] >> 16;
      const uint32_t lo1 = pv[1][e] & 0xffffu, hi1 = pv[1][e] >> 16;
      *reinterpret_cast<uint32_t*>(&sVt[buf][sub][vt_index(vd0 + 2 * e, kin)]) = lo0 | (lo1 << 16);
      *reinterpret_cast<uint32_t*>(&sVt[buf][sub][vt_index(vd0 + 2 * e + 1, kin)]) = hi0 | (hi1 << 16);
    }
  };

  const int pm = l32;
  const int pi_row = 16 * ((pm >> 3) >> 1) + 8 * ((pm >> 2) & 1) + 4 * ((pm >> 3) & 1) + (pm & 3);
  f32x16 acc_o[2];
#pragma unroll
  for (int x = 0; x < 16; ++x) acc_o[0][x] = acc_o[1][x] = 0.f;
  float m_run = 0.f, l_part[4] = {0.f, 0.f, 0.f, 0.f};
  op_t pprev[2];
  bool seen = false;

  gload(0);
  lstore(0);
  __syncthreads();
  for (int t = 0; t <= n_tiles; ++t) {
    const int buf = t % kNumBuf;
    if (t + 1 < n_tiles) gload(t + 1);
    const bool do_s = t < n_tiles && (KS * t + kh) * kBS < a.Lk;
    const bool do_pv = t >= 1 && (KS * (t - 1) + kh) * kBS < a.Lk;
    f32x16 sacc;
    mfma_priority<1>();
    if (do_s) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const op_t ka = __builtin_bit_cast(
            op_t, *reinterpret_cast<const u32x4*>(&sK[buf][(kh * 32 + pi_row) * kPitchK + ks * 16 + hl * 8]));
        sacc = Mfma<T>::run(ka, qreg[ks], ks == 0 ? f32x16{} : sacc);
      }
    }
    if (do_pv) {
      const int bufp = (t - 1) % kNumBuf;
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const op_t va = __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(
              &sVt[bufp][kh >> 1][vt_index(db * 32 + l32, (kh & 1) * 32 + ch * 16 + hl * 8)]));
          acc_o[db] = Mfma<T>::run(va, pprev[ch], acc_o[db]);
        }
    }
    mfma_priority<0>();
    if (do_s) {
      const int k0 = (KS * t + kh) * kBS;
      if (k0 + kBS > a.Lk) {
#pragma unroll
        for (int x = 0; x < 16; ++x)
          if (k0 + 16 * (x >> 3) + 8 * hl + (x & 7) >= a.Lk) sacc[x] = -INFINITY;
      }
      float m4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        m4[j] = fmaxf(fmaxf(sacc[4 * j], sacc[4 * j + 1]), fmaxf(sacc[4 * j + 2], sacc[4 * j + 3]));
      const float mx = half_swap_max(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]))) - m_run;
      const bool first = !seen;
      if (__any(first || mx > kTau)) {
        asm volatile("" ::: "memory");
        const float delta = first ? mx : fmaxf(mx, 0.f);
        m_run += delta;
        if (!first) {
          const float alpha = fast_exp2(-delta);
#pragma unroll
          for (int j = 0; j < 4; ++j) l_part[j] *= alpha;
#pragma unroll
          for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int x = 0; x < 16; ++x) acc_o[db][x] *= alpha;
        }
      }
      seen = true;
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = fast_exp2(sacc[ch * 8 + 2 * e] - m_run);
          const float p1 = fast_exp2(sacc[ch * 8 + 2 * e + 1] - m_run);
          w[e] = Mfma<T>::pack(p0, p1);
          l_part[e] = l_part[e] + p0 + p1;
        }
        pprev[ch] = __builtin_bit_cast(op_t, w);
      }
    }
    if (t + 1 < n_tiles) {
      lstore((t + 1) % kNumBuf);
      __syncthreads();
    }
  }

  // ---- merge the four quarters of each group (the tile buffers are free after this barrier) ----
  const float lsum = (l_part[0] + l_part[1]) + (l_part[2] + l_part[3]);
  __syncthreads();
  if (kh != 0) {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int x = 0; x < 16; ++x) smerge[grp][kh - 1][db * 16 + x][lane] = acc_o[db][x];
    smerge[grp][kh - 1][32][lane] = seen ? m_run : -INFINITY;
    smerge[grp][kh - 1][33][lane] = lsum;
  }
  __syncthreads();
  if (kh != 0) return;
  float mq[KS], aq[KS];
  mq[0] = m_run;  // quarter 0 always sees key 0
  float m = m_run;
#pragma unroll
  for (int j = 1; j < KS; ++j) {
    mq[j] = smerge[grp][j - 1][32][lane];
    m = fmaxf(m, mq[j]);
  }
  float lq = 0.f;
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    aq[j] = fast_exp2(mq[j] - m);
    lq += (j == 0 ? lsum : smerge[grp][j - 1][33][lane]) * aq[j];
  }
  const float inv = 1.f / (lq + __shfl_xor(lq, 32));
  const int qi = q_wave + l32;
  if (qi < a.Lq) {
    e_t* orow = O + qi * a.os[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = db * 32 + i * 8 + hl * 4;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int x = i * 4 + r;
          float acc = acc_o[db][x] * aq[0];
#pragma unroll
          for (int j = 1; j < KS; ++j) acc += smerge[grp][j - 1][db * 16 + x][lane] * aq[j];
          v[r] = acc * inv;
        }
        u32x2 w;
        w[0] = Mfma<T>::pack(v[0], v[1]);
        w[1] = Mfma<T>::pack(v[2], v[3]);
        *reinterpret_cast<u32x2*>(orow + d) = w;
      }
  }
}

// Causal / generic kernel shape: 32-query wavefronts, 8 per workgroup.
constexpr int kQB = 1;
constexpr int kNW = 8;

// The hand-scheduled kernel when its items fill the chip and its query blocks are mostly full
// (padding <= 15% of the rows): 384-query items (the encoder's 1500 = 4 x 384 - 36), else
// 256-query items (the DTW decoder's 448, a prompt's 224). Non-causal, 16-bit. Returns whether it
// launched.
template <typename T>
bool launch_pipe(const DenseArgs& a, hipStream_t stream) {
  const int64_t lim = 0x7fffffff, bh = (int64_t)a.B * a.H;
  const bool offs32 = (int64_t)a.Lk * a.ks[2] * 2 < lim && (int64_t)a.Lk * a.vs[2] * 2 < lim &&
                      (int64_t)a.Lq * a.qs[2] * 2 < lim && (int64_t)a.Lq * a.os[2] * 2 < lim;
  auto fits = [&](int64_t bm) {
    const int64_t items = bh * ((a.Lq + bm - 1) / bm);
    return (a.Lq + bm - 1) / bm * bm * 100 <= (int64_t)a.Lq * 115 && items >= kNumCus && items <= lim;
  };
  if (a.causal || a.Lk < kPMinKeys || !offs32) return false;
  if (fits(32 * 3 * kPWaves)) {
    // persistent: one workgroup per CU, each taking every 256th item
    hipLaunchKernelGGL((dense_pipe_kernel<T, 3>), dim3((unsigned)kNumCus), dim3(kPThreads), 0, stream, a);
    return true;
  }
  if (fits(32 * 2 * kPWaves)) {
    hipLaunchKernelGGL((dense_pipe_kernel<T, 2>), dim3((unsigned)kNumCus), dim3(kPThreads), 0, stream, a);
    return true;
  }
  return false;
}

template <typename T>
hipError_t launch_typed(const DenseArgs& a, hipStream_t stream) {
  if (!a.causal) {
    // One workgroup per CU is what each kernel is shaped for. Small grids (a single window, the
    // DTW decoder at B=1) take the key-split kernel with the largest query block that still
    // yields no more workgroups than CUs; the rest the 512-query kernel.
    // A launch of the 512-query kernel whose last round would hold few workgroups hands the
    // heads of that round to the key-split kernel instead (a second launch that has the whole
    // chip): the DTW decoder's 448 x 1500 cross-attention at B=16 is 256 + 64 heads.
    const int64_t bh = (int64_t)a.B * a.H;
    const int64_t q1 = (a.Lq + 127) / 128, q2 = (a.Lq + 255) / 256, qf = (a.Lq + kFBM - 1) / kFBM;
    const int64_t n = bh * qf;
    if (n <= 0) return hipSuccess;
    if (n > 0x7fffffff) return hipErrorInvalidValue;
    auto split = [&](const DenseArgs& s, int64_t heads) {
      if (heads * q1 <= kNumCus)
        hipLaunchKernelGGL((dense_split4_kernel<T>), dim3((unsigned)(heads * q1)), dim3(1024), 0, stream, s);
      else
        hipLaunchKernelGGL((dense_split_kernel<T, 2>), dim3((unsigned)(heads * q2)), dim3(512), 0, stream, s);
    };
    if (bh * q2 <= kNumCus) {
      split(a, bh);
      return hipGetLastError();
    }
    if (launch_pipe<T>(a, stream)) return hipGetLastError();
    const int64_t bh_main = (n / kNumCus) * kNumCus / qf;  // heads filling whole rounds
    const int64_t bh_rest = bh - bh_main;
    if (bh_main > 0 && bh_rest > 0 && bh_rest * q2 <= kNumCus && bh_rest * qf * 2 <= kNumCus) {
      hipLaunchKernelGGL((dense_fwd_kernel<T>), dim3((unsigned)(bh_main * qf)), dim3(kFThreads), 0, stream, a);
      DenseArgs rest = a;
      rest.bh0 = (int)bh_main;
      split(rest, bh_rest);
      return hipGetLastError();
    }
    hipLaunchKernelGGL((dense_fwd_kernel<T>), dim3((unsigned)n), dim3(kFThreads), 0, stream, a);
    return hipGetLastError();
  }
  constexpr int kBM = 32 * kQB * kNW;
  const int n_qblk = (a.Lq + kBM - 1) / kBM;
  const int64_t n = (int64_t)a.B * a.H * n_qblk;
  if (n <= 0) return hipSuccess;
  if (n > 0x7fffffff) return hipErrorInvalidValue;
  if (a.causal)
    hipLaunchKernelGGL((dense_mfma_kernel<T, true, kQB, kNW>), dim3((unsigned)n), dim3(kNW * 64), 0, stream, a);
  else
    hipLaunchKernelGGL((dense_mfma_kernel<T, false, kQB, kNW>), dim3((unsigned)n), dim3(kNW * 64), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_kv_prefill(int dtype, const KvArgs& a, hipStream_t stream) {
  if (a.kn == nullptr && (dtype == 1 || dtype == 2)) {
    // cross-attention over whole cache rows: the dense hand-scheduled kernel with the slot map
    // (strides here in elements: DenseArgs orders them b, h, row)
    DenseArgs d{};
    d.q = a.q;
    d.k = a.kc;
    d.v = a.vc;
    d.o = a.o;
    d.B = a.B;
    d.H = a.H;
    d.Lq = a.sq;
    d.Lk = a.Lk;
    d.causal = 0;
    d.bh0 = 0;
    const int64_t qs[3] = {a.qs[0], a.qs[2], a.qs[1]}, ks[3] = {a.kcs[0], a.kcs[2], a.kcs[1]};
    const int64_t vs[3] = {a.vcs[0], a.vcs[2], a.vcs[1]}, os[3] = {a.os[0], a.os[2], a.os[1]};
    bool aligned = true;
    for (int i = 0; i < 3; ++i) {
      aligned = aligned && qs[i] % 2 == 0 && ks[i] % 2 == 0 && vs[i] % 2 == 0 && os[i] % 2 == 0;
      d.qs[i] = qs[i] / 2;
      d.ks[i] = ks[i] / 2;
      d.vs[i] = vs[i] / 2;
      d.os[i] = os[i] / 2;
    }
    d.c = a.c;
    d.slot = a.bidx;
    d.n_slots = a.n_slots;
    const bool ok = aligned && (dtype == 2 ? launch_pipe<Bf16>(d, stream) : launch_pipe<F16>(d, stream));
    if (ok) return hipGetLastError();
  }
  const int n_qblk = (a.sq + 255) / 256;
  const dim3 grid((unsigned)(a.B * n_qblk), (unsigned)a.H);
  const bool has_new = a.kn != nullptr;
  if (dtype == 2) {
    if (has_new) hipLaunchKernelGGL((kv_prefill_kernel<Bf16, true>), grid, dim3(512), 0, stream, a);
    else hipLaunchKernelGGL((kv_prefill_kernel<Bf16, false>), grid, dim3(512), 0, stream, a);
  } else if (dtype == 1) {
    if (has_new) hipLaunchKernelGGL((kv_prefill_kernel<F16, true>), grid, dim3(512), 0, stream, a);
    else hipLaunchKernelGGL((kv_prefill_kernel<F16, false>), grid, dim3(512), 0, stream, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dense_mfma(int dtype, const DenseArgs& a, hipStream_t stream) {
  if (dtype == 1) return launch_typed<F16>(a, stream);
  if (dtype == 2) return launch_typed<Bf16>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace wdrz
