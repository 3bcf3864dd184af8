// attn_dense.hip — flash-style dense attention on CDNA4 bf16/fp16 MFMA (gfx950).
//
// Replaces F.scaled_dot_product_attention at reference src/whisperdrz/model.py:288-296
// (encoder self-attention, [B, 20, 1500, 64], non-causal, scale 1/8; and the uncached decoder,
// top-left causal). O = softmax(scale * Q K^T) V per (b, h), with an online softmax in the
// log2 domain.
//
// Layout of the work. A workgroup of 8 wavefronts owns 256 query rows of one (b, h); each
// wavefront owns 32 of them, which keeps it at ~120 VGPRs so four wavefronts share a SIMD and
// hide each other's MFMA, LDS and exp latencies. Key/value tiles of 64 rows are staged through
// LDS (three buffers: the global loads of tile t+1 are in flight while tile t is computed, one
// barrier per tile). Each tile is consumed as two 32-key sub-steps.
//
// Transposed products. The wavefront computes S^T = K Q^T with v_mfma_f32_32x32x16 (A = K from
// LDS, B = Q kept in registers), so a lane owns whole query COLUMNS of S: the row max and row
// sum are in-lane work plus one exchange between the two 32-lane halves, and the output rescale
// is per lane. The output is produced transposed too, O^T = V^T P^T (A = V^T from LDS, B = P
// straight from the S accumulators). For P to serve as the B operand without shuffles, the K
// rows feeding S^T are loaded in a permuted order so that accumulator a of lane l holds key
// 16*(a>>3) + 8*(l>>5) + (a&7) of its 32-key block: accumulators 8c..8c+7 are then the eight
// consecutive keys the lane supplies for 16-key chunk c of the PV product, and the matching
// V^T operand is one 16-byte LDS read. V is transposed into LDS at staging time.
//
// VALU diet (at head_dim 64 the softmax VALU work rivals the MFMA work):
//   * Q is pre-scaled by scale*log2(e) once, so a score costs one subtract before exp2;
//     fmax runs without NaN canonicalisation (the file is built with -fno-honor-nans; masked
//     scores are -inf, never NaN).
//   * Lazy rescaling: the running max only moves when a score exceeds it by more than 2^kTau
//     (P values up to 2^8 are exact enough in bf16 and harmless in fp32 sums); in steady state
//     the output accumulator is never rescaled.
//   * Row sums use v_dot2_f32_{bf16,f16} on the packed 16-bit P against (1, 1): one
//     instruction per two scores, summing exactly the P that feeds the MFMA, into four
//     independent partial sums (no serial dependency chain).
// Within a sub-step the wavefront issues the S_s MFMAs, then the PV_{s-1} MFMAs, then the
// softmax of S_s, so its VALU work can run while the matrix pipe drains PV_{s-1}.
//
// Grid. One workgroup per (b, h, 256-query block), flattened and remapped so that the query
// blocks of one (b, h) land on the same XCD (work-group ids are dealt round-robin over the
// 8 XCDs): they then share K/V through that XCD's L2.
#include "wdrz_common.h"
#include "wdrz_launch.h"

#include <type_traits>

namespace wdrz {

namespace {

constexpr int kBN = 64;               // key rows per LDS tile
constexpr int kBS = 32;               // key rows per sub-step
constexpr int kPitchK = kHeadDim + 8; // K tile row pitch in elements (16-byte pad)
constexpr int kNumBuf = 3;            // LDS tile buffers
constexpr int kNumXcd = 8;
constexpr float kTau = 8.0f;          // lazy-rescale threshold (log2 units)

template <typename T> struct Mfma;
template <> struct Mfma<Bf16> {
  typedef bf16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
  static __device__ __forceinline__ float widen_lo(uint32_t w) { return bf16_lo(w); }
  static __device__ __forceinline__ float widen_hi(uint32_t w) { return bf16_hi(w); }
  // sum of the two packed values, accumulated into acc
  static __device__ __forceinline__ float dot_ones(uint32_t w, float acc) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    const v2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, w), one, acc, false);
  }
};
template <> struct Mfma<F16> {
  typedef f16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
  static __device__ __forceinline__ float widen_lo(uint32_t w) { return f16_lo(w); }
  static __device__ __forceinline__ float widen_hi(uint32_t w) { return f16_hi(w); }
  static __device__ __forceinline__ float dot_ones(uint32_t w, float acc) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    const v2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, w), one, acc, false);
  }
};

__device__ __forceinline__ int remap_xcd(int id, int n) {
  const int q = n / kNumXcd, rem = n % kNumXcd;
  const int xcd = id % kNumXcd, local = id / kNumXcd;
  return xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
}

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
  const int tile_id = remap_xcd(blockIdx.x, gridDim.x);
  const int qblk = tile_id % n_qblk;
  const int bh = tile_id / n_qblk;
  const int b = bh / a.H, h = bh % a.H;

  const e_t* Q = reinterpret_cast<const e_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const e_t* K = reinterpret_cast<const e_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const e_t* V = reinterpret_cast<const e_t*>(a.v) + b * a.vs[0] + h * a.vs[1];
  e_t* O = reinterpret_cast<e_t*>(a.o) + b * a.os[0] + h * a.os[1];

  const int q_wg = qblk * kBM;
  const int q_wave = q_wg + wave * 32 * QB;
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
            l_part[qb][e] = Mfma<T>::dot_ones(w[e], l_part[qb][e]);
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

// Workgroup shape: query blocks per wavefront and wavefronts per workgroup.
#ifndef WDRZ_DENSE_QB
#define WDRZ_DENSE_QB 1
#endif
#ifndef WDRZ_DENSE_NW
#define WDRZ_DENSE_NW 8
#endif
constexpr int kQB = WDRZ_DENSE_QB;
constexpr int kNW = WDRZ_DENSE_NW;

template <typename T>
hipError_t launch_typed(const DenseArgs& a, hipStream_t stream) {
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

hipError_t launch_dense_mfma(int dtype, const DenseArgs& a, hipStream_t stream) {
  if (dtype == 1) return launch_typed<F16>(a, stream);
  if (dtype == 2) return launch_typed<Bf16>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace wdrz
