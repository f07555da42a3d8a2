// Fused STFT: framing + reflect padding + window + FFT + onesided slice + (freq, time) layout in
// one kernel that reads the raw waveform (trnfft/api.py:291-365 materialises the padded signal,
// the frame matrix, the windowed frames and a zero imaginary plane before its per-frame c2c).
//
// The frames are real, so two of them share one complex transform: z = w*x_a + i*w*x_b gives
// X_a[k] = (Z[k] + conj(Z[n-k])) / 2 and X_b[k] = (Z[k] - conj(Z[n-k])) / (2i).
// One workgroup takes FR consecutive frames of one signal (FR/2 complex LDS transforms):
//   1. the samples the tile covers ((FR-1)*hop + n_fft, reflect-padded at the signal edges) are
//      staged into LDS with wide coalesced loads, the window too;
//   2. each frame pair is windowed out of LDS and transformed (LDS Stockham);
//   3. the spectra go to LDS; the two real spectra are separated there while lanes run over
//      consecutive frames, so every store instruction writes FR contiguous floats of one bin row
//      of the (batch, bins, frames) output.
#include "kernels.h"

namespace tfa {

// Launch shape from a sweep on MI355X (64 waveforms x 160000 samples, hop n_fft/2, buffers
// rotated past the Infinity Cache, n_fft 64..4096): E = 8 elements per thread (many lanes per
// transform) is fastest at every length, with 8192/n_fft frame pairs per workgroup (~70 KB of LDS,
// two workgroups per CU, 256..1024 threads); stft_epth (fft_shape.h) gives E.
template <int NFFT>
constexpr int stft_default_pairs() {
  constexpr int p = 8192 / NFFT;
  return p < 2 ? 2 : p > 32 ? 32 : p;
}
template <int NFFT, int PAIRS_ = stft_default_pairs<NFFT>(), int E_ = stft_epth(NFFT)>
struct StftCfg {
  static constexpr int E = E_;
  static constexpr int T = NFFT / E;
  static constexpr int PADN = lds_pad(NFFT) + 1;  // odd pitch: pair regions start on different banks
  static constexpr int PAIRS = PAIRS_;             // complex transforms per workgroup
  static constexpr int FR = 2 * PAIRS;             // frames per workgroup
  static constexpr int THREADS = PAIRS * T;
  static constexpr int LDSF = 2 * PAIRS * PADN;  // floats of the spectra area (also the staging area)
  // the spectra are interleaved (re, im) float2 entries: PADN per pair
  static_assert((long long)LDSF * 4 + NFFT * 4 <= kLdsBytes, "STFT tile exceeds LDS");
  static_assert(THREADS > 0 && (FR & (FR - 1)) == 0, "frame tile must be a power of two");
};

// staging-area word of sample i of the tile span (one pad word per 32 spreads frame starts over banks)
__device__ __forceinline__ int stage_pad(int i) { return i + (i >> 5); }

template <int NFFT, int PAIRS = stft_default_pairs<NFFT>(), int E_ = stft_epth(NFFT)>
__global__ __launch_bounds__((StftCfg<NFFT, PAIRS, E_>::THREADS)) void stft_kernel(
    const float* __restrict__ sig, const float* __restrict__ win, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, int length, int hop, int pad,
    int n_frames, int n_bins, int tiles_per_signal, float scale) {
  using C = StftCfg<NFFT, PAIRS, E_>;
  constexpr int E = C::E, T = C::T, FR = C::FR, PADN = C::PADN, THREADS = C::THREADS;
  __shared__ float2 lds2[C::LDSF / 2];
  __shared__ float wl[NFFT];
  float* lds = reinterpret_cast<float*>(lds2);
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_signal;
  const int f0 = (int)(tile % tiles_per_signal) * FR;
  const int tid = threadIdx.x % T;
  const int pl = threadIdx.x / T;
  const int fa = f0 + 2 * pl;  // frames fa (real part) and fa + 1 (imaginary part)
  const float* x = sig + (size_t)b * length;

  for (int i = threadIdx.x; i < NFFT; i += THREADS) wl[i] = win[i];
  const int start = f0 * hop - pad;  // padded-signal origin of the tile's first frame
  const int span = (FR - 1) * hop + NFFT;
  float2 v[E];
  if (stage_pad(span) <= C::LDSF) {
    // 1. stage the span (block-uniform branch)
    if (start >= 0 && start + span <= length && ((reinterpret_cast<size_t>(x + start) & 15) == 0)) {
      const float4* src = reinterpret_cast<const float4*>(x + start);
      // three float4 loads in flight per thread before the LDS writes (a load-then-store loop waits
      // out the memory latency once per iteration): n_fft 256 64.8 -> 61.7 us, 1024 75.0 -> 73.4
      constexpr int U = 3;
      for (int q0 = threadIdx.x; q0 < span / 4; q0 += U * THREADS) {
        float4 s4[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int q = q0 + u * THREADS;
          if (q < span / 4) s4[u] = ld_stream4(src + q);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int q = q0 + u * THREADS;
          if (q < span / 4) {
            const int a = stage_pad(4 * q);  // 4q % 32 <= 28: the 4 words share one pad period
            lds[a] = s4[u].x;
            lds[a + 1] = s4[u].y;
            lds[a + 2] = s4[u].z;
            lds[a + 3] = s4[u].w;
          }
        }
      }
      for (int i = (span / 4) * 4 + threadIdx.x; i < span; i += THREADS) lds[stage_pad(i)] = x[start + i];
    } else {
      for (int i = threadIdx.x; i < span; i += THREADS) {
        int idx = start + i;
        // reflect without repeating the edge sample (torch.nn.functional.pad mode="reflect");
        // positions that only frames past the end would read are clamped (never stored)
        idx = idx < 0 ? -idx : idx;
        idx = idx >= length ? 2 * (length - 1) - idx : idx;
        idx = idx < 0 ? 0 : (idx >= length ? length - 1 : idx);
        lds[stage_pad(i)] = x[idx];
      }
    }
    __syncthreads();
    // 2. window the pair's two frames out of LDS
    const int oa = 2 * pl * hop;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int j = tid + T * e;
      const float w = wl[j];
      v[e] = make_float2(lds[stage_pad(oa + j)] * w, lds[stage_pad(oa + hop + j)] * w);
    }
    __syncthreads();  // the transform below reuses the staging area
  } else {
    // span too long for LDS (hop much larger than n_fft): per-frame loads
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int j = tid + T * e;
      const float w = win[j];
      float s[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int idx = (fa + h) * hop + j - pad;
        idx = idx < 0 ? -idx : idx;
        idx = idx >= length ? 2 * (length - 1) - idx : idx;
        idx = idx < 0 ? 0 : (idx >= length ? length - 1 : idx);
        s[h] = x[idx] * w;
      }
      v[e] = make_float2(s[0], s[1]);
    }
  }
  float2* my = lds2 + pl * PADN;
  LdsFft<NFFT, E, -1, (T <= 64), false, true, stft_pf(NFFT)>::run(v, reinterpret_cast<float*>(my), nullptr, tw, tid);
#pragma unroll
  for (int e = 0; e < E; ++e) my[lds_pad(tid + T * e)] = v[e];
  __syncthreads();
  // 3. lanes over consecutive frames fr: frame fr = 2p (+1) is the real (imaginary) part of pair p.
  //    Flat loop over (bin, frame) so any FR / THREADS ratio is covered; every iteration advances.
  const float hs = 0.5f * scale;
  const size_t ob = (size_t)b * n_bins * n_frames + f0;
  const int total = n_bins * FR;
  for (int i = threadIdx.x; i < total; i += THREADS) {
    const int fr = i % FR;
    const int k = i / FR;
    if (f0 + fr >= n_frames) continue;
    const float2* zp = lds2 + (fr >> 1) * PADN;
    const float2 z = zp[lds_pad(k)], y = zp[lds_pad((NFFT - k) & (NFFT - 1))];
    const float zr = z.x, zi = z.y, yr = y.x, yi = y.y;
    const bool odd = fr & 1;
    const float re = odd ? (zi + yi) : (zr + yr);
    const float im = odd ? (yr - zr) : (zi - yi);
    const size_t o = ob + (size_t)k * n_frames + fr;
    // plain (not streaming) stores: a workgroup's row segments rarely start on a cache line,
    // and L2 merges the partial lines the neighbouring workgroups write (measured 1.4x faster)
    out_re[o] = re * hs;
    out_im[o] = im * hs;
  }
}

template <int NFFT>
static hipError_t launch_stft_n(const StftArgs& a) {
  using C = StftCfg<NFFT>;
  const int tiles = (a.n_frames + C::FR - 1) / C::FR;
  const long long blocks = a.batch * (long long)tiles;
  hipLaunchKernelGGL((stft_kernel<NFFT>), dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream, a.signal, a.window,
                     a.out_re, a.out_im, a.tw, a.length, a.hop, a.pad, a.n_frames, a.n_bins, tiles, a.scale);
  return hipGetLastError();
}

hipError_t launch_stft(int n_fft, const StftArgs& a) {
  switch (n_fft) {
    case 16: return launch_stft_n<16>(a);
    case 32: return launch_stft_n<32>(a);
    case 64: return launch_stft_n<64>(a);
    case 128: return launch_stft_n<128>(a);
    case 256: return launch_stft_n<256>(a);
    case 512: return launch_stft_n<512>(a);
    case 1024: return launch_stft_n<1024>(a);
    case 2048: return launch_stft_n<2048>(a);
    case 4096: return launch_stft_n<4096>(a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfa
