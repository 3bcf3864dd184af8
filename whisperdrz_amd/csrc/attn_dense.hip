// attn_dense.hip — flash-style dense attention on CDNA4 bf16/fp16 MFMA (gfx950).
//
// Replaces F.scaled_dot_product_attention at reference src/whisperdrz/model.py:288-296
// (encoder self-attention, [B, 20, 1500, 64], non-causal, scale 1/8; and the uncached decoder,
// top-left causal). O = softmax(c' * Q K^T) V per (b, h), computed with an online softmax in
// the log2 domain (c = scale * log2 e).
//
// Tiling. A workgroup of 4 wavefronts owns 256 query rows of one (b, h); each wavefront owns
// 64 of them (two 32-row blocks). Key/value tiles of 64 rows are staged through LDS (double
// buffered, register prefetch of the next tile while the current one is in the MFMAs).
//
// The wavefront computes S^T = K Q^T with v_mfma_f32_32x32x16 (A = K from LDS, B = Q held in
// registers for the whole kernel), so every lane owns whole query COLUMNS of S: the row max
// and row sum of the softmax are in-lane work plus one exchange with lane ^ 32, and the
// rescale of the output accumulator is per-lane. The output is produced transposed as well,
// O^T = V^T P^T (A = V^T from LDS, B = P straight from the S accumulators after exp2 and
// conversion to 16 bits). For P to be usable as the B operand without any shuffle, the K rows
// feeding S^T are loaded in a permuted order pi(m) chosen so that accumulator a of lane l
// holds key 16*(a>>3) + 8*(l>>5) + (a&7) of its 32-key block; accumulators 8c..8c+7 of a lane
// are then exactly the eight consecutive keys that lane must supply for the 16-key chunk c of
// the PV product, and the matching V^T operand is one 16-byte LDS read.
//
// Grid. One workgroup per (b, h, 256-query block), flattened and remapped so that the query
// blocks of one (b, h) land on the same XCD (work-group ids are dealt round-robin over the
// 8 XCDs): they then share K/V through that XCD's L2.
#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {

namespace {

constexpr int kWavesD = 4;
constexpr int kThreadsD = kWavesD * 64;
constexpr int kBM = 64 * kWavesD;  // query rows per workgroup
constexpr int kBN = 64;            // key rows per tile
constexpr int kPitch = kHeadDim + 8;  // LDS row pitch in elements (16-byte pad)
constexpr int kNumXcd = 8;

template <typename T> struct Mfma;
template <> struct Mfma<Bf16> {
  typedef bf16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
};
template <> struct Mfma<F16> {
  typedef f16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
};

__device__ __forceinline__ int remap_xcd(int id, int n) {
  const int q = n / kNumXcd, rem = n % kNumXcd;
  const int xcd = id % kNumXcd, local = id / kNumXcd;
  return xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
}

template <typename T, bool CAUSAL>
__global__ __launch_bounds__(kThreadsD, 2) void dense_mfma_kernel(DenseArgs a) {
  typedef typename Mfma<T>::op_t op_t;
  typedef uint16_t e_t;
  __shared__ __attribute__((aligned(16))) e_t sK[2][kBN * kPitch];
  __shared__ __attribute__((aligned(16))) e_t sVt[2][kHeadDim * kPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hl = lane >> 5;  // lane half
  const int l32 = lane & 31;

  const int n_qblk = (a.Lq + kBM - 1) / kBM;
  const int tile = remap_xcd(blockIdx.x, gridDim.x);
  const int qblk = tile % n_qblk;
  const int bh = tile / n_qblk;
  const int b = bh / a.H, h = bh % a.H;

  const e_t* Q = reinterpret_cast<const e_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const e_t* K = reinterpret_cast<const e_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const e_t* V = reinterpret_cast<const e_t*>(a.v) + b * a.vs[0] + h * a.vs[1];
  e_t* O = reinterpret_cast<e_t*>(a.o) + b * a.os[0] + h * a.os[1];

  const int q_wg = qblk * kBM;
  const int q_wave = q_wg + wave * 64;

  // Q operand (B of S^T = K Q^T): lane holds query q_wave + qb*32 + l32, dims ks*16 + hl*8 + 0..7.
  op_t qreg[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = min(q_wave + qb * 32 + l32, a.Lq - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qreg[qb][ks] = __builtin_bit_cast(op_t, load16(Q + qi * a.qs[2] + ks * 16 + hl * 8));
  }

  // Keys needed by this workgroup.
  int k_lim = a.Lk;
  if (CAUSAL) k_lim = min(a.Lk, q_wg + kBM);
  const int n_tiles = (k_lim + kBN - 1) / kBN;

  // Tile loader: thread owns key pair (2*kp, 2*kp+1) and dims d0..d0+7 of each.
  const int kp = tid >> 3;
  const int d0 = (tid & 7) * 8;
  u32x4 pk[2], pv[2];
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = min(kt * kBN + 2 * kp + i, a.Lk - 1);
      pk[i] = load16(K + key * a.ks[2] + d0);
      pv[i] = load16(V + key * a.vs[2] + d0);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<u32x4*>(&sK[buf][(2 * kp + i) * kPitch + d0]) = pk[i];
    // V^T: element (d, key) at d*kPitch + key; pack the key pair into one dword.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo0 = pv[0][e] & 0xffffu, hi0 = pv[0][e] >> 16;
      const uint32_t lo1 = pv[1][e] & 0xffffu, hi1 = pv[1][e] >> 16;
      *reinterpret_cast<uint32_t*>(&sVt[buf][(d0 + 2 * e) * kPitch + 2 * kp]) = lo0 | (lo1 << 16);
      *reinterpret_cast<uint32_t*>(&sVt[buf][(d0 + 2 * e + 1) * kPitch + 2 * kp]) = hi0 | (hi1 << 16);
    }
  };

  // Permuted key row this lane feeds as the A operand of S^T (see header comment).
  const int pm = l32;
  const int pi_row = 16 * ((pm >> 3) >> 1) + 8 * ((pm >> 2) & 1) + 4 * ((pm >> 3) & 1) + (pm & 3);

  f32x16 acc_o[2][2];  // [db][qb]: O^T rows d = db*32 + ..., column = query
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) acc_o[i][j][x] = 0.f;
  float m_run[2] = {kNegBig, kNegBig};
  float l_run[2] = {0.f, 0.f};
  const float c = a.c;

  if (n_tiles > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();

  for (int kt = 0; kt < n_tiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < n_tiles) gload(kt + 1);
    const int k0 = kt * kBN;
    bool active = true;
    if (CAUSAL) active = k0 <= q_wave + 63;
    if (active) {
      // ---- S^T = K Q^T ----
      f32x16 s[2][2];  // [kb][qb]
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int x = 0; x < 16; ++x) s[kb][qb][x] = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const op_t ka = __builtin_bit_cast(
              op_t, *reinterpret_cast<const u32x4*>(&sK[buf][(kb * 32 + pi_row) * kPitch + ks * 16 + hl * 8]));
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) s[kb][qb] = Mfma<T>::run(ka, qreg[qb][ks], s[kb][qb]);
        }
      }
      // ---- mask (tail tile, causal diagonal) ----
      const bool need_mask = (k0 + kBN > a.Lk) || (CAUSAL && k0 + kBN - 1 > q_wave);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            const int qi = q_wave + qb * 32 + l32;
#pragma unroll
            for (int x = 0; x < 16; ++x) {
              const int key = k0 + kb * 32 + 16 * (x >> 3) + 8 * hl + (x & 7);
              bool ok = key < a.Lk;
              if (CAUSAL) ok = ok && key <= qi;
              if (!ok) s[kb][qb][x] = -INFINITY;
            }
          }
      }
      // ---- online softmax per query column ----
      op_t pop[2][4];  // [qb][chunk]: B operand of O^T = V^T P^T
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        float mx = s[0][qb][0];
#pragma unroll
        for (int x = 1; x < 16; ++x) mx = fmaxf(mx, s[0][qb][x]);
#pragma unroll
        for (int x = 0; x < 16; ++x) mx = fmaxf(mx, s[1][qb][x]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run[qb], mx);
        const float alpha = fast_exp2((m_run[qb] - m_new) * c);
        m_run[qb] = m_new;
        const float mc = m_new * c;
        float ps = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float p0 = fast_exp2(__builtin_fmaf(s[kb][qb][half * 8 + 2 * e], c, -mc));
              const float p1 = fast_exp2(__builtin_fmaf(s[kb][qb][half * 8 + 2 * e + 1], c, -mc));
              ps += p0 + p1;
              w[e] = Mfma<T>::pack(p0, p1);
            }
            pop[qb][kb * 2 + half] = __builtin_bit_cast(op_t, w);
          }
        }
        l_run[qb] = __builtin_fmaf(l_run[qb], alpha, ps);
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int x = 0; x < 16; ++x) acc_o[db][qb][x] *= alpha;
      }
      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const op_t va = __builtin_bit_cast(
              op_t, *reinterpret_cast<const u32x4*>(&sVt[buf][(db * 32 + l32) * kPitch + kc * 16 + hl * 8]));
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) acc_o[db][qb] = Mfma<T>::run(va, pop[qb][kc], acc_o[db][qb]);
        }
      }
    }
    if (kt + 1 < n_tiles) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and store: lane holds query column, 4 consecutive dims per (db, i) ----
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float lt = l_run[qb] + __shfl_xor(l_run[qb], 32);
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

template <typename T>
hipError_t launch_typed(const DenseArgs& a, hipStream_t stream) {
  const int n_qblk = (a.Lq + kBM - 1) / kBM;
  const int64_t n = (int64_t)a.B * a.H * n_qblk;
  if (n <= 0) return hipSuccess;
  if (n > 0x7fffffff) return hipErrorInvalidValue;
  if (a.causal)
    hipLaunchKernelGGL((dense_mfma_kernel<T, true>), dim3((unsigned)n), dim3(kThreadsD), 0, stream, a);
  else
    hipLaunchKernelGGL((dense_mfma_kernel<T, false>), dim3((unsigned)n), dim3(kThreadsD), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_dense_mfma(int dtype, const DenseArgs& a, hipStream_t stream) {
  if (dtype == 1) return launch_typed<F16>(a, stream);
  if (dtype == 2) return launch_typed<Bf16>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace wdrz
