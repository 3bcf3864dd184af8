// linear.hip — the decode step's MLP input projection with its activation fused:
// Y = GELU(X W^T + b) for the first two modules of ResidualAttentionBlock.mlp
// (src/whisperdrz/model.py:388-391, Linear(n_state, 4 n_state) then nn.GELU(), applied at
// model.py:434). The reference runs a library GEMM with a bias epilogue, rounds the result to
// the 16-bit type, and then a separate elementwise GELU (exact, erf form) rounds again; this
// kernel does the same arithmetic (fp32 accumulation, bias in fp32, rounding to the storage
// type, GELU in fp32, rounding) in one launch, so the [rows, 4 n_state] pre-activation never
// goes through memory.
//
// Shape: decode-step rows are few (a batch bucket, <= 64), so the product is bound by reading
// W (4 n_state x n_state 16-bit values) and by the latency of that stream. One 256-thread
// workgroup computes a 64-row x 16 NJ-feature block over K in chunks of 128: each chunk of W
// (16 NJ x 128) and X (64 x 128) is loaded with whole 256-byte row segments per 16 lanes (full
// cache lines) and written to one of two LDS buffers; wavefront
// w then runs v_mfma_f32_16x16x32 on rows 16w .. 16w + 15 from LDS, so no partial sums cross
// wavefronts and the epilogue works on its own accumulators. W is cold (read once per decode
// step, 13 MB per layer at large-v3): each thread requests its whole share of up to ten chunks
// at once, so the grid keeps nearly all of W in flight; X, just written and in L2, runs a
// shorter register pipeline a few chunks ahead. Feature rows past N re-read the
// last valid row (clamped) and are not stored; rows past M are not loaded, computed or stored.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {
namespace {

template <typename T> struct LinMfma;
template <> struct LinMfma<Bf16> {
  typedef bf16x8 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float round(float v) { return (float)(__bf16)v; }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
};
template <> struct LinMfma<F16> {
  typedef f16x8 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float round(float v) { return (float)(_Float16)v; }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
};

__device__ __forceinline__ float gelu_erf(float v) { return 0.5f * v * (1.f + erff(v * 0.70710678118654752f)); }

constexpr int kLinRows = 64;    // rows (M) per workgroup
constexpr int kLinChunk = 128;  // K per LDS stage
constexpr int kLinPad = 8;      // 16-bit elements of row padding in LDS (16 bytes)
constexpr int kLinLd = kLinChunk + kLinPad;
constexpr int kLinWChunks = 10;  // chunks of W requested together (K = 1280 in one group)

// PART: split-K form. Workgroup z of grid dimension z covers K range [z Kc, (z + 1) Kc), Kc =
// K / n_split, and stores its fp32 partial sums (no bias, no rounding, no activation) to
// part[z][m][n]; the consumer adds the splits and the bias.
template <typename T, int ACT, int NJ, int kLinPf, bool PART>
__global__ __launch_bounds__(256) void linear_act_kernel(LinearArgs a) {
  typedef typename LinMfma<T>::op_t op_t;
  constexpr int kLinFeat = 16 * NJ;  // output features (N) per workgroup
  __shared__ __align__(16) uint16_t sW[2][kLinFeat][kLinLd];
  __shared__ __align__(16) uint16_t sX[2][kLinRows][kLinLd];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * kLinFeat, m0 = blockIdx.y * kLinRows;

  // loader: thread t copies 16 bytes at K offset 8 (t % 16) of rows t / 16 + 16 q
  const int lr = tid >> 4, lk = (tid & 15) * 8;
  const int k_len = PART ? a.K / a.n_split : a.K;
  const int k_base = PART ? (int)blockIdx.z * k_len : 0;
  const uint16_t* W = static_cast<const uint16_t*>(a.w) + k_base;
  const uint16_t* X = static_cast<const uint16_t*>(a.x) + k_base;
  const uint16_t* wsrc[NJ];
  const uint16_t* xsrc[4];
#pragma unroll
  for (int q = 0; q < NJ; ++q) wsrc[q] = W + (int64_t)min(n0 + lr + 16 * q, a.N - 1) * a.w_stride + lk;
#pragma unroll
  for (int q = 0; q < 4; ++q) xsrc[q] = X + (int64_t)min(m0 + lr + 16 * q, a.M - 1) * a.x_stride + lk;
  // rows past M are neither loaded nor stored (their LDS rows feed only their own outputs)
  const int rows = min(a.M - m0, kLinRows);

  const int n_chunks = k_len / kLinChunk;
  // X (just written by the previous kernel, in L2): kLinPf chunks ahead in registers
  u32x4 rx[kLinPf][4];
  auto fetch_x = [&](int c, u32x4* x4) {
    const int k = c * kLinChunk;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (lr + 16 * q < rows) x4[q] = load16(xsrc[q] + k);
  };
#pragma unroll
  for (int p = 0; p < kLinPf; ++p)
    if (p < n_chunks) fetch_x(p, rx[p]);

  // MFMA operands: lane holds 8 K values of row lane % 16 at K offset 8 (lane / 16)
  const int li = lane & 15, lq = (lane >> 4) * 8;
  f32x4 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  static_assert(kLinWChunks % kLinPf == 0, "register sets of X must line up across W groups");
  for (int c0 = 0; c0 < n_chunks; c0 += kLinWChunks) {
    // W (cold, streamed from HBM): every chunk of this group requested at once, so the whole
    // grid keeps ~all of W in flight instead of a latency-bound trickle
    u32x4 rw[kLinWChunks][NJ];
#pragma unroll
    for (int i = 0; i < kLinWChunks; ++i)
      if (c0 + i < n_chunks)
#pragma unroll
        for (int q = 0; q < NJ; ++q) rw[i][q] = load16_stream(wsrc[q] + (c0 + i) * kLinChunk);
#pragma unroll
    for (int i = 0; i < kLinWChunks; ++i) {
      const int c = c0 + i;
      if (c < n_chunks) {
        const int buf = c & 1, p = i % kLinPf;
        // buf was last read by the compute of chunk c - 2, which every wavefront finished
        // before the barrier of chunk c - 1
#pragma unroll
        for (int q = 0; q < NJ; ++q) *reinterpret_cast<u32x4*>(&sW[buf][lr + 16 * q][lk]) = rw[i][q];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (lr + 16 * q < rows) *reinterpret_cast<u32x4*>(&sX[buf][lr + 16 * q][lk]) = rx[p][q];
        if (c + kLinPf < n_chunks) fetch_x(c + kLinPf, rx[p]);
        __syncthreads();
        if (16 * wave < rows) {
#pragma unroll
          for (int ks = 0; ks < kLinChunk / 32; ++ks) {
            const op_t xb =
                __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(&sX[buf][16 * wave + li][32 * ks + lq]));
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              const op_t wa =
                  __builtin_bit_cast(op_t, *reinterpret_cast<const u32x4*>(&sW[buf][16 * j + li][32 * ks + lq]));
              acc[j] = LinMfma<T>::run(wa, xb, acc[j]);
            }
          }
        }
      }
    }
  }

  // acc[j] lane holds C[n = 16 j + 4 (lane / 16) + r][m = 16 wave + lane % 16], r = 0..3
  const int m = m0 + 16 * wave + li;
  if (m >= a.M) return;
  if constexpr (PART) {
    float* P = a.part + ((int64_t)blockIdx.z * a.M + m) * a.N;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int nb = n0 + 16 * j + (lane >> 4) * 4;
      if (nb < a.N) *reinterpret_cast<f32x4*>(P + nb) = acc[j];
    }
    return;
  }
  const uint16_t* B = static_cast<const uint16_t*>(a.bias);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int nb = n0 + 16 * j + (lane >> 4) * 4;
    if (nb >= a.N) continue;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float s = acc[j][r];
      if (B) s += __is_same(T, Bf16) ? bf16_lo(B[nb + r]) : f16_lo(B[nb + r]);
      s = LinMfma<T>::round(s);  // the Linear's output in the storage type, as the reference has it
      v[r] = ACT ? gelu_erf(s) : s;
    }
    uint2 out;
    out.x = LinMfma<T>::pack(v[0], v[1]);
    out.y = LinMfma<T>::pack(v[2], v[3]);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.y) + (int64_t)m * a.y_stride + nb) = out;
  }
}

}  // namespace

template <typename T, int NJ, int PF>
void launch_t(const LinearArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((a.N + 16 * NJ - 1) / (16 * NJ)), (unsigned)((a.M + kLinRows - 1) / kLinRows),
                  (unsigned)(a.part ? a.n_split : 1));
  if (a.part) hipLaunchKernelGGL((linear_act_kernel<T, 0, NJ, PF, true>), grid, dim3(256), 0, stream, a);
  else if (a.act) hipLaunchKernelGGL((linear_act_kernel<T, 1, NJ, PF, false>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((linear_act_kernel<T, 0, NJ, PF, false>), grid, dim3(256), 0, stream, a);
}

hipError_t launch_linear(int dtype, const LinearArgs& a, hipStream_t stream) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  // 16 features per workgroup, X two chunks ahead; 32 features once 16 would give 320 or more
  // workgroups (more than one per CU). Measured at 64 rows, 32 cold weights in a graph: fc1
  // (5120 x 1280) 10.8 -> 10.1 us and fc2's split-K quarters (1280 x 5120) 10.3 -> 9.5 us with 32;
  // the q/k/v projection (240 workgroups) 8.3 vs 9.9 us and the output projections' halves (160)
  // 4.9 vs 5.7 us stay on 16; 64 features per workgroup is slower everywhere.
  const int64_t wgs16 = (int64_t)((a.N + 15) / 16) * ((a.M + kLinRows - 1) / kLinRows) * (a.part ? a.n_split : 1);
  if (wgs16 >= 320) {
    if (dtype == 2) launch_t<Bf16, 2, 2>(a, stream);
    else launch_t<F16, 2, 2>(a, stream);
  } else {
    if (dtype == 2) launch_t<Bf16, 1, 2>(a, stream);
    else launch_t<F16, 1, 2>(a, stream);
  }
  return hipGetLastError();
}

}  // namespace wdrz
