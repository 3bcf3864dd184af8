// attn_kvcache.hip — split-KV attention for the decoder's cached paths (gfx950).
//
// Replaces flash_attn_with_kvcache / _sdpa_attn_with_kvcache (reference
// src/whisperdrz/model.py:20-95) for:
//   * cached self-attention with fused in-place append of k_new / v_new (model.py:49-63):
//     query t of batch row b sees keys j <= cache_seqlens[b] + t (bottom-right causal);
//   * cross-attention over the full cache (model.py:64-67), non-causal;
// and also serves as the fp32 dense SDPA kernel (model.py:288-296, top-left causal flag).
//
// Work decomposition. One workgroup (256 lanes) per (batch row b, query block, head h, split).
// The decode work is a GEMV per (b, h): every key row is touched once, so the kernel is HBM
// bound and uses no MFMA. A head row of K or V is 64 elements = one 16-byte load per lane
// across LPK lanes (8 lanes in 16-bit types, 16 in fp32); the workgroup's 256/LPK lane groups
// each own a strided subset of the split's keys, keep U keys in flight per batch, and run an
// online softmax in the log2 domain. Group partials are merged with shuffles inside a
// wavefront and through LDS across the four wavefronts. When several splits share a
// (b, t, h) row they write (m, l, o) partials to the caller's workspace and a combine pass
// merges them.
//
// Append: keys at positions >= cache_seqlens[b] are read straight from k_new / v_new, never
// from the cache, so the in-place write (done by the split whose key range holds the row)
// cannot race with any read in the same launch.
#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSQ = 8;  // query rows per workgroup
constexpr int kUnroll = 4; // keys per lane group per batch (even: P V runs on key pairs)
constexpr float kTau = 8.0f;  // lazy-rescale threshold (log2 units)

// v_dot2 on packed 16-bit pairs with fp32 accumulation.
template <typename T> struct Dot2;
template <> struct Dot2<Bf16> {
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  static constexpr uint32_t kOnes = 0x3f803f80u;  // (1.0, 1.0)
  static __device__ __forceinline__ float run(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
};
template <> struct Dot2<F16> {
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static constexpr uint32_t kOnes = 0x3c003c00u;  // (1.0, 1.0)
  static __device__ __forceinline__ float run(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
};

template <typename T, int SQ, bool HAS_NEW>
__global__ __launch_bounds__(kThreads) void kv_attn_kernel(KvArgs a) {
  constexpr int EB = ElemBytes<T>::value;
  constexpr int EPL = 16 / EB;         // elements per lane per 16-byte load
  constexpr int LPK = kHeadDim / EPL;  // lanes per key row
  constexpr int G = kThreads / LPK;    // key groups per workgroup

  __shared__ float sm_acc[kWaves][SQ][kHeadDim];
  __shared__ float sm_m[kWaves][SQ];
  __shared__ float sm_l[kWaves][SQ];

  const int tid = threadIdx.x;
  const int g = tid / LPK;
  const int r = tid % LPK;
  const int wave = tid / 64;
  const int lane = tid % 64;

  const int b = blockIdx.x / a.n_qblocks;
  const int t0 = (blockIdx.x % a.n_qblocks) * SQ;
  const int h = blockIdx.y;
  const int split = blockIdx.z;
  const int nq = min(SQ, a.sq - t0);

  const int slot = a.bidx ? a.bidx[b] : b;
  const int cs = HAS_NEW ? a.seqlens[b] : 0;
  // Metadata the host cannot validate without reading device memory. A bad row produces NaN
  // output instead of touching memory outside the cache.
  const bool bad = slot < 0 || slot >= a.n_slots || cs < 0 || (HAS_NEW && cs + a.sq > a.Lk);

  // Keys this query block needs: [0, key_lim).
  int key_lim;
  if (HAS_NEW)
    key_lim = cs + t0 + nq;
  else if (a.causal)
    key_lim = min(a.Lk, t0 + nq);
  else
    key_lim = a.Lk;
  const int k_begin = split * a.split_len;
  const int k_end = bad ? k_begin : min(key_lim, k_begin + a.split_len);

  // Queries. 16-bit types keep the raw packed pairs for v_dot2 (the scale is applied to the
  // reduced score); fp32 keeps floats pre-scaled into the log2 domain.
  u32x4 qraw[SQ];
  float qf[SQ][EPL];
#pragma unroll
  for (int t = 0; t < SQ; ++t) {
    const int tt = t0 + min(t, nq - 1);
    qraw[t] = load16(a.q + b * a.qs[0] + tt * a.qs[1] + h * a.qs[2] + r * 16);
    if constexpr (EB == 4) {
      Slice<T> sl;
      sl.from_raw(qraw[t]);
#pragma unroll
      for (int e = 0; e < EPL; ++e) qf[t][e] = sl.v[e] * a.c;
    }
  }

  // Per query: running max (log2 units), partial row sum and output slice of this lane group.
  float m[SQ], l[SQ], acc[SQ][EPL];
#pragma unroll
  for (int t = 0; t < SQ; ++t) {
    m[t] = kNegBig;
    l[t] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[t][e] = 0.f;
  }
  // Last key each query may see inside this split (inclusive).
  int lim[SQ];
#pragma unroll
  for (int t = 0; t < SQ; ++t) {
    lim[t] = k_end - 1;
    if (HAS_NEW) lim[t] = min(lim[t], cs + t0 + t);
    else if (a.causal) lim[t] = min(lim[t], t0 + t);
  }

  const int safe_slot = bad ? 0 : slot;
  const char* kc_row = a.kc + safe_slot * a.kcs[0] + h * a.kcs[2] + r * 16;
  const char* vc_row = a.vc + safe_slot * a.vcs[0] + h * a.vcs[2] + r * 16;
  const char* kn_row = HAS_NEW ? a.kn + b * a.kns[0] + h * a.kns[2] + r * 16 : nullptr;
  const char* vn_row = HAS_NEW ? a.vn + b * a.vns[0] + h * a.vns[2] + r * 16 : nullptr;

  for (int base = k_begin + g; base < k_end; base += G * kUnroll) {
    u32x4 kr[kUnroll], vr[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int kk = min(base + u * G, k_end - 1);
      const char* kp;
      const char* vp;
      if (HAS_NEW && kk >= cs) {
        kp = kn_row + (int64_t)(kk - cs) * a.kns[1];
        vp = vn_row + (int64_t)(kk - cs) * a.vns[1];
      } else {
        kp = kc_row + (int64_t)kk * a.kcs[1];
        vp = vc_row + (int64_t)kk * a.vcs[1];
      }
      kr[u] = load16(kp);
      vr[u] = load16(vp);
    }
    // ---- scores (log2 units), masked to -inf outside each query's key range ----
    float sc[SQ][kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if constexpr (EB == 2) {
#pragma unroll
        for (int t = 0; t < SQ; ++t) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) d = Dot2<T>::run(qraw[t][i], kr[u][i], d);
          sc[t][u] = group_sum<LPK>(d) * a.c;
        }
      } else {
        Slice<T> ks;
        ks.from_raw(kr[u]);
#pragma unroll
        for (int t = 0; t < SQ; ++t) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < EPL; ++e) d = __builtin_fmaf(qf[t][e], ks.v[e], d);
          sc[t][u] = group_sum<LPK>(d);
        }
      }
#pragma unroll
      for (int t = 0; t < SQ; ++t)
        if (base + u * G > lim[t]) sc[t][u] = -INFINITY;
    }
    // ---- lazy max update: move the reference only when a score exceeds it by > kTau ----
    float mb[SQ];
    bool grow = false;
#pragma unroll
    for (int t = 0; t < SQ; ++t) {
      mb[t] = sc[t][0];
#pragma unroll
      for (int u = 1; u < kUnroll; ++u) mb[t] = fmaxf(mb[t], sc[t][u]);
      grow = grow || mb[t] > m[t] + kTau;
    }
    if (__any(grow)) {
#pragma unroll
      for (int t = 0; t < SQ; ++t) {
        const float mn = mb[t] > m[t] + kTau ? mb[t] : m[t];
        const float alpha = fast_exp2(m[t] - mn);
        m[t] = mn;
        l[t] *= alpha;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[t][e] *= alpha;
      }
    }
    // ---- P V ----
    if constexpr (EB == 2) {
      // Keys in pairs: v_perm gathers dim e of both keys into one dword, v_dot2 multiplies it
      // with the packed pair of probabilities.
#pragma unroll
      for (int u = 0; u < kUnroll; u += 2) {
        u32x4 vlo, vhi;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          vlo[i] = __builtin_amdgcn_perm(vr[u + 1][i], vr[u][i], 0x05040100u);
          vhi[i] = __builtin_amdgcn_perm(vr[u + 1][i], vr[u][i], 0x07060302u);
        }
#pragma unroll
        for (int t = 0; t < SQ; ++t) {
          const uint32_t pp = Dot2<T>::pack(fast_exp2(sc[t][u] - m[t]), fast_exp2(sc[t][u + 1] - m[t]));
          l[t] = Dot2<T>::run(pp, Dot2<T>::kOnes, l[t]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[t][2 * i] = Dot2<T>::run(pp, vlo[i], acc[t][2 * i]);
            acc[t][2 * i + 1] = Dot2<T>::run(pp, vhi[i], acc[t][2 * i + 1]);
          }
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        Slice<T> vs;
        vs.from_raw(vr[u]);
#pragma unroll
        for (int t = 0; t < SQ; ++t) {
          const float p = fast_exp2(sc[t][u] - m[t]);
          l[t] += p;
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[t][e] = __builtin_fmaf(p, vs.v[e], acc[t][e]);
        }
      }
    }
  }

  // In-place append of this block's new rows that fall in this split's key range.
  if (HAS_NEW && !bad) {
    const int lo = split * a.split_len, hi = lo + a.split_len;
    for (int idx = tid; idx < nq * 2 * LPK; idx += kThreads) {
      const int t = idx / (2 * LPK);
      const int which = (idx / LPK) & 1;
      const int rr = idx % LPK;
      const int pos = cs + t0 + t;
      if (pos >= lo && pos < hi) {
        if (which == 0)
          store16(a.kc + slot * a.kcs[0] + (int64_t)pos * a.kcs[1] + h * a.kcs[2] + rr * 16,
                  load16(a.kn + b * a.kns[0] + (int64_t)(t0 + t) * a.kns[1] + h * a.kns[2] +
                         rr * 16));
        else
          store16(a.vc + slot * a.vcs[0] + (int64_t)pos * a.vcs[1] + h * a.vcs[2] + rr * 16,
                  load16(a.vn + b * a.vns[0] + (int64_t)(t0 + t) * a.vns[1] + h * a.vns[2] +
                         rr * 16));
      }
    }
  }

  // Merge lane groups inside the wavefront (groups differ in lane bits >= log2(LPK)).
#pragma unroll
  for (int off = LPK; off < 64; off *= 2) {
#pragma unroll
    for (int t = 0; t < SQ; ++t) {
      const float mo = __shfl_xor(m[t], off);
      const float lo = __shfl_xor(l[t], off);
      const float mn = fmaxf(m[t], mo);
      const float fa = fast_exp2(m[t] - mn), fb = fast_exp2(mo - mn);
      l[t] = l[t] * fa + lo * fb;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[t][e] = acc[t][e] * fa + __shfl_xor(acc[t][e], off) * fb;
      m[t] = mn;
    }
  }
  if (lane < LPK) {
#pragma unroll
    for (int t = 0; t < SQ; ++t) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) sm_acc[wave][t][r * EPL + e] = acc[t][e];
      if (r == 0) {
        sm_m[wave][t] = m[t];
        sm_l[wave][t] = l[t];
      }
    }
  }
  __syncthreads();

  for (int idx = tid; idx < nq * kHeadDim; idx += kThreads) {
    const int t = idx / kHeadDim, d = idx % kHeadDim;
    float mm = kNegBig;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sm_m[w][t]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(sm_m[w][t] - mm);
      L = __builtin_fmaf(sm_l[w][t], f, L);
      O = __builtin_fmaf(sm_acc[w][t][d], f, O);
    }
    const int tt = t0 + t;
    if (a.n_splits == 1) {
      const float val = bad ? __builtin_nanf("") : O / L;
      char* op = a.o + b * a.os[0] + tt * a.os[1] + h * a.os[2];
      if constexpr (EB == 4)
        reinterpret_cast<float*>(op)[d] = val;
      else if constexpr (__is_same(T, Bf16))
        reinterpret_cast<__bf16*>(op)[d] = (__bf16)val;
      else
        reinterpret_cast<_Float16*>(op)[d] = (_Float16)val;
    } else {
      const int64_t row = ((int64_t)b * a.sq + tt) * a.H + h;
      float* p = a.ws + (row * a.n_splits + split) * (kHeadDim + 2);
      p[d] = O;
      if (d == 0) {
        p[kHeadDim] = bad ? __builtin_nanf("") : mm;
        p[kHeadDim + 1] = L;
      }
    }
  }
}

// Merge the per-split partials of one (b, t, h) row: grid (sq, H, B), 64 lanes (one per d).
template <typename T>
__global__ __launch_bounds__(64) void kv_combine_kernel(KvArgs a) {
  const int d = threadIdx.x;
  const int t = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t row = ((int64_t)b * a.sq + t) * a.H + h;
  const float* p = a.ws + row * a.n_splits * (kHeadDim + 2);
  float mm = kNegBig;
  for (int s = 0; s < a.n_splits; ++s) mm = fmaxf(mm, p[s * (kHeadDim + 2) + kHeadDim]);
  float L = 0.f, O = 0.f;
  for (int s = 0; s < a.n_splits; ++s) {
    const float* ps = p + s * (kHeadDim + 2);
    const float f = fast_exp2(ps[kHeadDim] - mm);
    L = __builtin_fmaf(ps[kHeadDim + 1], f, L);
    O = __builtin_fmaf(ps[d], f, O);
  }
  const float val = O / L;
  char* op = a.o + b * a.os[0] + t * a.os[1] + h * a.os[2];
  if constexpr (ElemBytes<T>::value == 4)
    reinterpret_cast<float*>(op)[d] = val;
  else if constexpr (__is_same(T, Bf16))
    reinterpret_cast<__bf16*>(op)[d] = (__bf16)val;
  else
    reinterpret_cast<_Float16*>(op)[d] = (_Float16)val;
}

template <typename T>
hipError_t launch_typed(const KvArgs& a, hipStream_t stream) {
  dim3 grid(a.B * a.n_qblocks, a.H, a.n_splits);
  const bool has_new = a.kn != nullptr;
  const int sq_blk = a.n_qblocks > 1 ? kMaxSQ : a.sq;
#define WDRZ_KV_CASE(SQV)                                                                   \
  case SQV:                                                                                 \
    if (has_new)                                                                            \
      hipLaunchKernelGGL((kv_attn_kernel<T, SQV, true>), grid, dim3(kThreads), 0, stream, a); \
    else                                                                                    \
      hipLaunchKernelGGL((kv_attn_kernel<T, SQV, false>), grid, dim3(kThreads), 0, stream, a); \
    break;
  switch (sq_blk) {
    WDRZ_KV_CASE(1)
    WDRZ_KV_CASE(2)
    WDRZ_KV_CASE(3)
    WDRZ_KV_CASE(4)
    WDRZ_KV_CASE(5)
    WDRZ_KV_CASE(6)
    WDRZ_KV_CASE(7)
    WDRZ_KV_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef WDRZ_KV_CASE
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  if (a.n_splits > 1) {
    hipLaunchKernelGGL((kv_combine_kernel<T>), dim3(a.sq, a.H, a.B), dim3(64), 0, stream, a);
    err = hipGetLastError();
  }
  return err;
}

}  // namespace

void kv_split_plan(int64_t units, int64_t Lk, int* n_splits, int* split_len) {
  // Aim for >= 1024 workgroups (four per CU on 256 CUs) while keeping >= 64 keys per split.
  const int64_t max_splits = (Lk + 63) / 64;
  int64_t want = (1024 + units - 1) / (units > 0 ? units : 1);
  if (want < 1) want = 1;
  if (want > max_splits) want = max_splits;
  int64_t len = (Lk + want - 1) / want;
  len = (len + 63) / 64 * 64;
  if (len < 64) len = 64;
  *split_len = (int)len;
  *n_splits = (int)((Lk + len - 1) / len);
  if (*n_splits < 1) *n_splits = 1;
}

size_t kv_workspace_bytes(int64_t B, int64_t sq, int64_t H, int n_splits) {
  if (n_splits <= 1) return 0;
  return (size_t)(B * sq * H) * (size_t)n_splits * (kHeadDim + 2) * sizeof(float);
}

hipError_t launch_kv_attn(int dtype, const KvArgs& a, hipStream_t stream) {
  switch (dtype) {
    case 0:
      return launch_typed<F32>(a, stream);
    case 1:
      return launch_typed<F16>(a, stream);
    case 2:
      return launch_typed<Bf16>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace wdrz
