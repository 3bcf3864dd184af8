// attn_dense_f32.hip — dense attention in fp32 on the fp32 matrix cores (gfx950).
//
// Replaces F.scaled_dot_product_attention at reference src/whisperdrz/model.py:288-296 when the
// model runs in fp32 (the reference's CPU-runnable configuration: one encoder layer B=1 H=20
// L=1500 D=64, and the uncached decoder with a top-left causal mask). O = softmax(scale Q K^T) V
// per (b, h), online softmax in the log2 domain, fp32 throughout.
//
// Both products run on v_mfma_f32_32x32x2_f32 (32x32 output, K = 2 per instruction, lane halves
// h = lane / 32 supplying the two K slots):
//   * S^T = K Q^T per 32-key step: 32 MFMAs over the 64 head dims. The K slot of lane half h at
//     instruction kk is head dim 32h + kk, for K (A operand, row = key lane % 32) and Q (B
//     operand, column = query lane % 32) alike, so each lane reads 32 contiguous floats of its
//     K row (eight 16-byte LDS reads) and keeps its 32 Q floats in registers. Two accumulator
//     chains (even / odd kk) keep the matrix pipe busy.
//   * O^T += V^T P^T: 16 MFMAs per 32 output dims. Accumulator i = 4j + r of lane l holds key
//     8j + 4h + r of S^T, so at instruction kk = i both operands use that key in K slot h: P is
//     the accumulator itself (no shuffles) and V^T is one 4-byte LDS read of row 8j + 4h + r.
// At 64 MFMAs of 64 cycles per step against ~150 VALU instructions of softmax, the kernel is
// bound by the fp32 matrix rate. A 512-thread workgroup holds four 32-query groups, each served
// by two wavefronts on the same SIMD that take alternate 32-key steps (so every SIMD has two
// wavefronts to cover each other's stalls) and merge their (m, l, O) through LDS at the end.
// 64-key K and V stages go through registers into three LDS buffers (two stages ahead), one
// barrier per stage; each wavefront issues its next step's S^T before its own softmax, and the
// output is rescaled only when a row max grows.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {
namespace {

constexpr int kF32Groups = 4;                 // 32-query groups per workgroup
constexpr int kF32Waves = 2 * kF32Groups;     // two key halves per group
constexpr int kF32Threads = kF32Waves * 64;
constexpr int kF32BM = 32 * kF32Groups;  // queries per workgroup
constexpr int kF32BS = 32;               // keys per step (one wavefront)
constexpr int kF32Stage = 2 * kF32BS;    // keys per LDS stage (both halves)
constexpr int kF32Pitch = kHeadDim + 4;  // LDS row pitch in floats (16-byte pad: conflict-free b128 reads)

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <bool CAUSAL>
__global__ __launch_bounds__(kF32Threads) void dense_f32_kernel(DenseArgs a) {
  __shared__ __attribute__((aligned(16))) float sK[3][kF32Stage * kF32Pitch];
  __shared__ __attribute__((aligned(16))) float sV[3][kF32Stage * kF32Pitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = wave % kF32Groups;  // query group
  const int kh = wave / kF32Groups;  // key half: steps 2u + kh of each 64-key stage u
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  const int n_qblk = (a.Lq + kF32BM - 1) / kF32BM;
  const int tile_id = remap_xcd(blockIdx.x, gridDim.x);
  const int qblk = tile_id % n_qblk;
  const int bh = tile_id / n_qblk;
  const int b = bh / a.H, h = bh % a.H;

  const float* Q = static_cast<const float*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const float* K = static_cast<const float*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const float* V = static_cast<const float*>(a.v) + b * a.vs[0] + h * a.vs[1];
  float* O = static_cast<float*>(a.o) + b * a.os[0] + h * a.os[1];
  const int q_blk0 = qblk * kF32BM;
  const int q_wave0 = q_blk0 + qg * 32;
  const int q_me = q_wave0 + l32;  // this lane's query (may be >= Lq: computed, not stored)

  // Keys the workgroup and this wavefront need (top-left causal: query i sees keys 0..i).
  const int k_lim = CAUSAL ? min(a.Lk, q_blk0 + kF32BM) : a.Lk;
  const int k_lim_w = CAUSAL ? min(a.Lk, q_wave0 + 32) : a.Lk;
  const int n_units = (k_lim + kF32Stage - 1) / kF32Stage;

  // Q: 32 floats (head dims 32h .. 32h + 31) of this lane's query, pre-scaled by c.
  float qreg[32];
  {
    const float* qp = Q + (int64_t)min(q_me, a.Lq - 1) * a.qs[2] + 32 * hl;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f32x4 v = __builtin_bit_cast(f32x4, load16(qp + 4 * i));
#pragma unroll
      for (int e = 0; e < 4; ++e) qreg[4 * i + e] = v[e] * a.c;
    }
  }

  // Tile staging: thread t moves 16-byte pieces t and t + 512 of the 64 x 64 K and V tiles.
  u32x4 rk[2], rv[2];
  auto gload = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int piece = tid + i * kF32Threads;
      const int key = min(st * kF32Stage + (piece >> 4), a.Lk - 1);
      const int col = (piece & 15) * 4;
      rk[i] = load16(K + (int64_t)key * a.ks[2] + col);
      rv[i] = load16(V + (int64_t)key * a.vs[2] + col);
    }
  };
  auto lstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int piece = tid + i * kF32Threads;
      const int off = (piece >> 4) * kF32Pitch + (piece & 15) * 4;
      *reinterpret_cast<u32x4*>(&sK[buf][off]) = rk[i];
      *reinterpret_cast<u32x4*>(&sV[buf][off]) = rv[i];
    }
  };

  f32x16 acc_o[2];  // [db]: O^T rows d = 32 db + 8j + 4h + r, column = query
#pragma unroll
  for (int x = 0; x < 16; ++x) acc_o[0][x] = acc_o[1][x] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // S^T of step st (K tile in buffer buf), two accumulator chains summed at the end
  auto scores = [&](int buf, f32x16& out) __attribute__((always_inline)) {
    f32x16 sa, sb;
#pragma unroll
    for (int x = 0; x < 16; ++x) sa[x] = sb[x] = 0.f;
    const float* kr = &sK[buf][(kh * kF32BS + l32) * kF32Pitch + 32 * hl];
#pragma unroll
    for (int kq = 0; kq < 8; ++kq) {
      const f32x4 kv = *reinterpret_cast<const f32x4*>(kr + 4 * kq);
      sa = mfma_f32(kv[0], qreg[4 * kq + 0], sa);
      sb = mfma_f32(kv[1], qreg[4 * kq + 1], sb);
      sa = mfma_f32(kv[2], qreg[4 * kq + 2], sa);
      sb = mfma_f32(kv[3], qreg[4 * kq + 3], sb);
    }
#pragma unroll
    for (int x = 0; x < 16; ++x) out[x] = sa[x] + sb[x];
  };
  // online softmax of step st on sc (P written back into sc)
  auto softmax = [&](int st, f32x16& sc) __attribute__((always_inline)) {
    const int k0 = st * kF32BS;
    if (k0 + kF32BS > a.Lk || (CAUSAL && k0 + kF32BS - 1 > q_wave0)) {
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const int key = k0 + 8 * (x >> 2) + 4 * hl + (x & 3);
        if (key >= a.Lk || (CAUSAL && key > q_me)) sc[x] = -INFINITY;
      }
    }
    float mx = sc[0];
#pragma unroll
    for (int x = 1; x < 16; ++x) mx = fmaxf(mx, sc[x]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if (__any(mx > m_run)) {  // some row's max grows: rescale what was accumulated
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);  // 0 on the first step (m_run = -inf)
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        acc_o[0][x] *= alpha;
        acc_o[1][x] *= alpha;
      }
    }
    float psum = 0.f;
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      sc[x] = fast_exp2(sc[x] - m_run);
      psum += sc[x];
    }
    l_run += psum;
  };
  // O^T += V^T P^T: instruction i uses key 8(i>>2) + 4h + (i&3) in K slot h
  auto pv = [&](int buf, const f32x16& p) __attribute__((always_inline)) {
    const float* vr = &sV[buf][(kh * kF32BS + 4 * hl) * kF32Pitch + l32];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float* row = vr + (8 * (i >> 2) + (i & 3)) * kF32Pitch;
      acc_o[0] = mfma_f32(row[0], p[i], acc_o[0]);
      acc_o[1] = mfma_f32(row[32], p[i], acc_o[1]);
    }
  };

  // Stages of 64 keys (the two halves' steps) go two stages ahead into three buffers: at the top
  // of stage u, stages u and u+1 are visible, so S of the wavefront's step in stage u+1 is
  // issued before its softmax of stage u and the matrix pipe has work while the softmax runs.
  gload(0);
  lstore(0);
  if (n_units > 1) {
    gload(1);
    lstore(1);
  }
  if (n_units > 2) gload(2);
  __syncthreads();
  auto live = [&](int u) { return (2 * u + kh) * kF32BS < k_lim_w; };  // causal: keys end earlier
  f32x16 s_cur, s_nxt;
  if (live(0)) scores(0, s_cur);
  auto unit = [&](int u, f32x16& cur, f32x16& nxt) __attribute__((always_inline)) {
    if (live(u)) {
      if (u + 1 < n_units && live(u + 1)) scores((u + 1) % 3, nxt);
      softmax(2 * u + kh, cur);
      pv(u % 3, cur);
    }
    // Buffer (u+2)%3 last held stage u-1, whose reads (K in stage u-2, V in stage u-1) came
    // before the previous barrier.
    if (u + 2 < n_units) {
      lstore((u + 2) % 3);
      if (u + 3 < n_units) gload(u + 3);
    }
    __syncthreads();
  };
  int u = 0;
  for (; u + 1 < n_units; u += 2) {
    unit(u, s_cur, s_nxt);
    unit(u + 1, s_nxt, s_cur);
  }
  if (u < n_units) unit(u, s_cur, s_nxt);

  // ---- merge the two key halves of each query group through LDS (the tile area is free: the
  // last stage ended with a barrier), then normalise and store ----
  float* mg = &sK[0][0] + qg * (34 * 64);  // [34][64]: acc_o (32), m, l per lane
  if (kh == 1) {
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      mg[x * 64 + lane] = acc_o[0][x];
      mg[(16 + x) * 64 + lane] = acc_o[1][x];
    }
    mg[32 * 64 + lane] = m_run;
    mg[33 * 64 + lane] = l_run;
  }
  __syncthreads();
  if (kh == 1 || q_me >= a.Lq) return;
  const float m1 = mg[32 * 64 + lane];
  const float m = fmaxf(m_run, m1);  // finite: half 0 always sees key 0
  const float a0 = fast_exp2(m_run - m), a1 = fast_exp2(m1 - m);
  const float l_me = l_run * a0 + mg[33 * 64 + lane] * a1;
  const float inv = 1.f / (l_me + __shfl_xor(l_me, 32));
  // lane holds dims 32 db + 8j + 4h + r (r = 0..3) of its query
  float* orow = O + (int64_t)q_me * a.os[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 w;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int x = 4 * j + r;
        w[r] = (acc_o[db][x] * a0 + mg[(16 * db + x) * 64 + lane] * a1) * inv;
      }
      store16(orow + 32 * db + 8 * j + 4 * hl, __builtin_bit_cast(u32x4, w));
    }
}

}  // namespace

hipError_t launch_dense_f32(const DenseArgs& a, hipStream_t stream) {
  const int n_qblk = (a.Lq + kF32BM - 1) / kF32BM;
  const int64_t n = (int64_t)a.B * a.H * n_qblk;
  if (n <= 0) return hipSuccess;
  if (n > 0x7fffffff) return hipErrorInvalidValue;
  if (a.causal)
    hipLaunchKernelGGL((dense_f32_kernel<true>), dim3((unsigned)n), dim3(kF32Threads), 0, stream, a);
  else
    hipLaunchKernelGGL((dense_f32_kernel<false>), dim3((unsigned)n), dim3(kF32Threads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace wdrz
