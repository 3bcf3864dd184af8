// logmel.hip — gfx950 kernels for Whisper's log-mel front end.
//
// Replaces LogMelSpectrogram (src/whisperdrz/audio.py:81-156), which the reference runs on the
// CPU per 30-s window (transcriber.py:1091-1092):
//   stft(n_fft 400, hop 160, periodic Hann, center + reflect padding) -> |X|^2 of all frames but
//   the last -> slaney mel filterbank (torchaudio MelScale, norm/mel_scale "slaney") ->
//   log10(max(mel, 1e-10)) -> max(log, max_over_window - 8) -> (x + 4) / 4 -> pad with -1.5 /
//   truncate to target_frames.
//
// Three launches:
//   logmel_init_kernel   the [201, n_mels] filterbank and the cosine / Hann tables (computed in
//                        double, stored fp32) and each window's running maximum, into the
//                        workspace
//   logmel_spec_kernel   one workgroup per (32 frames, window), 4 wavefronts. The frames' samples
//                        (overlapping by 240) are staged once in LDS with the reflect padding;
//                        the windowed DFT is a [32 frames x 400 samples] x [400 x 256 bins]
//                        product on the fp32 matrix cores (v_mfma_f32_32x32x2_f32: real and
//                        imaginary parts as two accumulators over the same A operand; cosines
//                        from a 400-entry LDS table indexed by i*k mod 400). The power spectrum
//                        goes to LDS, a second product [32 x 202] x [202 x n_mels] applies the
//                        filterbank, and log10 is stored with the window maximum folded in by
//                        an atomic max.
//   logmel_finish_kernel (max(x, max - 8) + 4) / 4, and -1.5 past the last frame.
// fp32 throughout, like the reference; the DFT sums 400 products per bin in fp32.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wdrz_common.h"
#include "wdrz_launch.h"

namespace wdrz {
namespace {

constexpr int kNfft = 400;
constexpr int kHop = 160;
constexpr int kBins = kNfft / 2 + 1;     // 201
constexpr int kBinTiles = 8;             // 256 bins computed (2 tiles per wavefront), 201 kept
constexpr int kFrames = 32;              // frames per workgroup
constexpr int kSeg = (kFrames - 1) * kHop + kNfft;  // 5360 samples
constexpr int kPPitch = 225;             // power tile pitch (odd: conflict-free column reads)
constexpr int kKMel = 202;               // filterbank rows incl. one zero row (K multiple of 2)
// Samples are stored with one pad float per 32 (position j + j/32): the 32 frames a wavefront
// reads at once are 160 samples apart, which would otherwise fall into 2 of the 64 LDS banks.
constexpr int kSegStored = kSeg + kSeg / 32 + 1;
__device__ __forceinline__ int seg_pos(int j) { return j + (j >> 5); }

typedef float f32x16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16v mfma32x2(float a, float b, f32x16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Ordered encoding of floats so that an unsigned max is a float max (negative values reversed).
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float order_val(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Slaney mel scale (3 mels per 200 Hz below 1 kHz, 27 mels per factor 6.4 above).
__device__ double hz_to_mel(double f) {
  const double f_sp = 200.0 / 3.0;
  if (f < 1000.0) return f / f_sp;
  return 1000.0 / f_sp + log(f / 1000.0) / (log(6.4) / 27.0);
}
__device__ double mel_to_hz(double m) {
  const double f_sp = 200.0 / 3.0, min_log_mel = 1000.0 / f_sp;
  if (m < min_log_mel) return f_sp * m;
  return 1000.0 * exp(log(6.4) / 27.0 * (m - min_log_mel));
}

// fb[k][m] (row k = frequency bin, kKMel rows, row 201 zero), the window maxima, and the
// cosine / Hann tables (400 entries each, computed in double).
__global__ __launch_bounds__(256) void logmel_init_kernel(LogMelArgs a) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx < a.B) a.gmax[idx] = order_key(-INFINITY);
  if (idx < kNfft) {
    double sn, c;
    sincospi(2.0 * idx / kNfft, &sn, &c);
    a.tables[idx] = (float)c;
    a.tables[kNfft + idx] = (float)(0.5 - 0.5 * c);  // periodic Hann
  }
  if (idx >= kKMel * a.n_mels) return;
  const int k = idx / a.n_mels, m = idx % a.n_mels;
  float v = 0.f;
  if (k < kBins) {
    const double mel_max = hz_to_mel(8000.0);
    const double f0 = mel_to_hz(mel_max * m / (a.n_mels + 1));
    const double f1 = mel_to_hz(mel_max * (m + 1) / (a.n_mels + 1));
    const double f2 = mel_to_hz(mel_max * (m + 2) / (a.n_mels + 1));
    const double f = 8000.0 * k / (kBins - 1);
    const double down = (f - f0) / (f1 - f0), up = (f2 - f) / (f2 - f1);
    double t = down < up ? down : up;
    t = t > 0.0 ? t : 0.0;
    v = (float)(t * 2.0 / (f2 - f0));
  }
  a.fb[idx] = v;
}

__global__ __launch_bounds__(256) void logmel_spec_kernel(LogMelArgs a) {
  const int b = blockIdx.y;
  const int f0 = blockIdx.x * kFrames;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tid = threadIdx.x;
  const int N = a.n_samples;

  static_assert(kSegStored <= kFrames * kPPitch, "sample buffer");
  __shared__ float seg_p[kFrames * kPPitch];  // samples during the DFT, then the power tile
  __shared__ float win[kNfft];
  __shared__ float ctab[kNfft];
  __shared__ uint32_t wmax[4];

  const float* x = a.audio + (int64_t)b * a.audio_stride;
  // Padded sample j of this tile is original sample 160*f0 + j - 200, reflected at both ends.
  for (int j = tid; j < kSeg; j += 256) {
    int o = kHop * f0 + j - kNfft / 2;
    if (o < 0) o = -o;
    if (o >= N) o = 2 * (N - 1) - o;
    o = o < 0 ? 0 : (o >= N ? N - 1 : o);  // frames past the end only
    seg_p[seg_pos(j)] = x[o];
  }
  for (int j = tid; j < kNfft; j += 256) {
    ctab[j] = a.tables[j];
    win[j] = a.tables[kNfft + j];
  }
  __syncthreads();

  // ---- windowed DFT: wave w computes bin tiles w and w + 4 for the 32 frames (tile 7 is past
  // the 201 bins; computing it keeps every wavefront on the same straight-line code) ----
  const int fr = lane & 31;  // frame of this lane's A element / bin of its B element
  const int kk = lane >> 5;  // which of the 2 samples of a step
  f32x16v re[2], im[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) re[u] = im[u] = f32x16v{};
  int idx[2], step[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int n = 32 * (wave + 4 * u) + fr;  // bin
    idx[u] = (kk * n) % kNfft;               // (i * n) mod 400 for i = kk
    step[u] = (2 * n) % kNfft;
  }
#pragma unroll 8
  for (int s = 0; s < kNfft / 2; ++s) {
    const int i = 2 * s + kk;
    const float av = seg_p[seg_pos(kHop * fr + i)] * win[i];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float c = ctab[idx[u]];
      int is = idx[u] + 300;  // sin(t) = cos(t - pi/2): index - 100 mod 400
      is = is >= kNfft ? is - kNfft : is;
      const float sn = ctab[is];
      re[u] = mfma32x2(av, c, re[u]);
      im[u] = mfma32x2(av, sn, im[u]);
      idx[u] += step[u];
      idx[u] = idx[u] >= kNfft ? idx[u] - kNfft : idx[u];
    }
  }
  __syncthreads();  // every wavefront is done with the samples: the buffer becomes the power tile
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int n = 32 * (wave + 4 * u) + fr;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = 8 * (e / 4) + 4 * kk + (e % 4);  // frame within the tile
      const float p = re[u][e] * re[u][e] + im[u][e] * im[u][e];
      if (n < kKMel) seg_p[row * kPPitch + n] = n < kBins ? p : 0.f;
    }
  }
  __syncthreads();

  // ---- filterbank: wave w computes mel tile w, [32 frames] x [32 mels] over 202 bins ----
  const int n_tiles = (a.n_mels + 31) / 32;
  float vmax = -INFINITY;
  if (wave < n_tiles) {
    const int mel = 32 * wave + fr;
    const int melc = mel < a.n_mels ? mel : a.n_mels - 1;
    f32x16v acc = f32x16v{};
#pragma unroll 8
    for (int s = 0; s < kKMel / 2; ++s) {
      const int k = 2 * s + kk;
      const float av = seg_p[fr * kPPitch + k];
      const float bv = a.fb[k * a.n_mels + melc];
      acc = mfma32x2(av, bv, acc);
    }
    float* out = a.out + (int64_t)b * a.os[0] + (int64_t)mel * a.os[1];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int f = f0 + 8 * (e / 4) + 4 * kk + (e % 4);
      const float lv = log10f(fmaxf(acc[e], 1e-10f));
      if (mel < a.n_mels && f < a.n_frames) {
        vmax = fmaxf(vmax, lv);
        if (f < a.out_frames) out[f] = lv;
      }
    }
  }
  // window maximum: wave, then workgroup, then one atomic (vector) per workgroup
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, o));
  if (lane == 0) wmax[wave] = order_key(vmax);
  __syncthreads();
  if (tid == 0) {
    uint32_t k = wmax[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) k = k > wmax[w] ? k : wmax[w];
    atomicMax(a.gmax + b, k);
  }
}

__global__ __launch_bounds__(256) void logmel_finish_kernel(LogMelArgs a) {
  const int b = blockIdx.z, m = blockIdx.y;
  const int f = blockIdx.x * 256 + threadIdx.x;
  if (f >= a.out_frames) return;
  float* p = a.out + (int64_t)b * a.os[0] + (int64_t)m * a.os[1] + f;
  if (f >= a.n_frames) {
    *p = -1.5f;  // audio.py:133-137
    return;
  }
  const float floor_v = order_val(a.gmax[b]) - 8.0f;
  *p = (fmaxf(*p, floor_v) + 4.0f) / 4.0f;
}

}  // namespace

// Workspace: filterbank [202, n_mels], cosine + Hann tables [2, 400], window maxima [B].
namespace {
size_t fb_bytes(int64_t n_mels) { return ((size_t)(kKMel * n_mels) * sizeof(float) + 255) / 256 * 256; }
constexpr size_t kTableBytes = 2 * kNfft * sizeof(float);
}  // namespace

size_t logmel_workspace_bytes(int64_t B, int64_t n_mels) {
  return fb_bytes(n_mels) + kTableBytes + (size_t)B * sizeof(uint32_t);
}

hipError_t launch_logmel(LogMelArgs a, void* ws, hipStream_t stream) {
  char* p = static_cast<char*>(ws);
  a.fb = reinterpret_cast<float*>(p);
  a.tables = reinterpret_cast<float*>(p + fb_bytes(a.n_mels));
  a.gmax = reinterpret_cast<uint32_t*>(p + fb_bytes(a.n_mels) + kTableBytes);
  int init_n = kKMel * a.n_mels > a.B ? kKMel * a.n_mels : a.B;
  init_n = init_n > kNfft ? init_n : kNfft;
  hipLaunchKernelGGL(logmel_init_kernel, dim3((init_n + 255) / 256), dim3(256), 0, stream, a);
  hipLaunchKernelGGL(logmel_spec_kernel, dim3((a.n_frames + kFrames - 1) / kFrames, a.B), dim3(256), 0, stream, a);
  hipLaunchKernelGGL(logmel_finish_kernel, dim3((a.out_frames + 255) / 256, a.n_mels, a.B), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace wdrz
