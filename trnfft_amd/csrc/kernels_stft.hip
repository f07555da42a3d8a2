// Fused STFT: framing + reflect padding + window + FFT + onesided slice + (freq, time) layout in
// one kernel that reads the raw waveform (trnfft/api.py:291-365, which materialises the padded
// signal, the frame matrix, the windowed frames and a zero imaginary plane before its c2c).
//
// One workgroup = FT consecutive frames of one signal.  Each frame is an LDS-resident Stockham
// transform of n_fft points (real input).  The spectra are then transposed through LDS so each
// store writes FT consecutive frames of one frequency row of the (batch, bins, frames) output.
#include "kernels.h"

namespace tfa {

template <int NFFT>
struct StftCfg {
  static constexpr int E = lds_epth(NFFT);
  static constexpr int T = NFFT / E;
  // frames per workgroup: fill 256..1024 threads within the LDS budget
  static constexpr int FT = (T >= 1024) ? 1 : ((1024 / T) > 16 ? 16 : (1024 / T));
  static constexpr int PADN = lds_pad(NFFT) + 1;  // +1: transposed reads hit distinct banks
  static constexpr int THREADS = FT * T;
  static_assert((long long)FT * PADN * 8 <= kLdsBytes, "STFT tile exceeds LDS");
};

template <int NFFT>
__global__ __launch_bounds__(StftCfg<NFFT>::THREADS) void stft_kernel(
    const float* __restrict__ sig, const float* __restrict__ win, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, int length, int hop, int pad,
    int n_frames, int n_bins, int tiles_per_signal, float scale) {
  using C = StftCfg<NFFT>;
  constexpr int E = C::E, T = C::T, FT = C::FT, PADN = C::PADN;
  __shared__ float lre[FT * PADN];
  __shared__ float lim[FT * PADN];
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_signal;
  const int f0 = (int)(tile % tiles_per_signal) * FT;
  const int tid = threadIdx.x % T;
  const int fl = threadIdx.x / T;
  const int f = f0 + fl;
  const float* x = sig + (size_t)b * length;

  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = tid + T * e;
    float s = 0.0f;
    if (f < n_frames) {
      int idx = f * hop + j - pad;
      // reflect (no edge repeat), as torch.nn.functional.pad(mode="reflect")
      idx = idx < 0 ? -idx : idx;
      idx = idx >= length ? 2 * (length - 1) - idx : idx;
      s = x[idx] * win[j];
    }
    v[e] = make_float2(s, 0.0f);
  }
  LdsFft<NFFT, E, -1, false>::run(v, lre + fl * PADN, lim + fl * PADN, tw, tid);
  // spectra -> LDS (frame-major), then read back frame-fastest for coalesced row stores
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = tid + T * e;
    lre[fl * PADN + lds_pad(k)] = v[e].x;
    lim[fl * PADN + lds_pad(k)] = v[e].y;
  }
  __syncthreads();
  const int fr = threadIdx.x % FT;
  const int q = threadIdx.x / FT;
  const int fo = f0 + fr;
  const size_t obase = (size_t)b * n_bins * n_frames + fo;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = q + T * e;
    if (k < n_bins && fo < n_frames) {
      const int idx = fr * PADN + lds_pad(k);
      out_re[obase + (size_t)k * n_frames] = lre[idx] * scale;
      out_im[obase + (size_t)k * n_frames] = lim[idx] * scale;
    }
  }
}

template <int NFFT>
static hipError_t launch_stft_n(const StftArgs& a) {
  using C = StftCfg<NFFT>;
  const int tiles = (a.n_frames + C::FT - 1) / C::FT;
  const long long blocks = a.batch * (long long)tiles;
  hipLaunchKernelGGL((stft_kernel<NFFT>), dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream,
                     a.signal, a.window, a.out_re, a.out_im, a.tw, a.length, a.hop, a.pad, a.n_frames,
                     a.n_bins, tiles, a.scale);
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
