// Fused STFT: framing + reflect padding + window + FFT + onesided slice + (freq, time) layout in
// one kernel that reads the raw waveform (trnfft/api.py:291-365 materialises the padded signal,
// the frame matrix, the windowed frames and a zero imaginary plane before its per-frame c2c).
//
// The frames are real, so two of them share one complex transform: z = w*x_a + i*w*x_b gives
// X_a[k] = (Z[k] + conj(Z[n-k])) / 2 and X_b[k] = (Z[k] - conj(Z[n-k])) / (2i).  One workgroup
// takes FR consecutive frames of one signal (FR/2 complex LDS transforms); the spectra go through
// LDS once more so the two real spectra are separated there and each store writes a run of FR
// consecutive frames of one frequency row of the (batch, bins, frames) output.
#include "kernels.h"

namespace tfa {

// Complex transforms (frame pairs) per workgroup: as many as 512 threads and the LDS allow (for
// n_fft = 512: 32 pairs = 64 frames, 256 B row segments, re+im planes in LDS).  A sweep on MI355X
// showed the time falling almost linearly with frames per workgroup (8 frames: 285 us, 64: 83 us
// for 64 x 160000 samples): short row segments of the (bins, frames) output are what cost.
template <int NFFT>
constexpr int stft_default_pairs() {
  constexpr int t = NFFT / lds_epth(NFFT);
  int p = t >= 512 ? 1 : 512 / t;
  while (p > 1 && (long long)p * (lds_pad(NFFT) + 1) * 8 > kLdsBytes) p /= 2;
  return p;
}

template <int NFFT, int PAIRS_ = stft_default_pairs<NFFT>(), bool SPLIT_ = false>
struct StftCfg {
  static constexpr int E = lds_epth(NFFT);
  static constexpr int T = NFFT / E;
  static constexpr int PADN = lds_pad(NFFT) + 1;  // odd pitch: pair regions start on different banks
  static constexpr int PAIRS = PAIRS_;       // complex transforms per workgroup
  static constexpr int FR = 2 * PAIRS;       // frames per workgroup
  static constexpr int THREADS = PAIRS * T;
  static constexpr int PLANES = SPLIT_ ? 1 : 2;  // LDS planes per pair
  static_assert((long long)PAIRS * PADN * 4 * PLANES <= kLdsBytes, "STFT tile exceeds LDS");
};

template <int NFFT, int PAIRS = stft_default_pairs<NFFT>(), bool SPLIT = false>
__global__ __launch_bounds__((StftCfg<NFFT, PAIRS, SPLIT>::THREADS)) void stft_kernel(
    const float* __restrict__ sig, const float* __restrict__ win, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, int length, int hop, int pad,
    int n_frames, int n_bins, int tiles_per_signal, float scale) {
  using C = StftCfg<NFFT, PAIRS, SPLIT>;
  constexpr int E = C::E, T = C::T, FR = C::FR, PADN = C::PADN;
  // SPLIT: one plane per pair, exchanges go re then im; else re and im planes side by side
  __shared__ float lds[C::PLANES * C::PAIRS * PADN];
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_signal;
  const int f0 = (int)(tile % tiles_per_signal) * FR;
  const int tid = threadIdx.x % T;
  const int pl = threadIdx.x / T;
  const int fa = f0 + 2 * pl;  // frames fa (real part) and fa + 1 (imaginary part)
  const float* x = sig + (size_t)b * length;

  // tile-uniform fast path: every sample of every frame of the tile lies inside the signal
  const int first = f0 * hop - pad;
  const int last = (f0 + FR - 1) * hop - pad + NFFT - 1;
  const bool interior = first >= 0 && last < length && f0 + FR <= n_frames;

  float2 v[E];
  if (interior) {
    const float* xa = x + fa * hop - pad + tid;
    const float* xb = xa + hop;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float w = win[tid + T * e];
      v[e] = make_float2(xa[T * e] * w, xb[T * e] * w);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int j = tid + T * e;
      const float w = win[j];
      float s[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int f = fa + h;
        s[h] = 0.0f;
        if (f < n_frames) {
          int idx = f * hop + j - pad;
          // reflect without repeating the edge sample (torch.nn.functional.pad mode="reflect")
          idx = idx < 0 ? -idx : idx;
          idx = idx >= length ? 2 * (length - 1) - idx : idx;
          s[h] = x[idx] * w;
        }
      }
      v[e] = make_float2(s[0], s[1]);
    }
  }
  float* my = lds + pl * PADN;
  float* my_im = SPLIT ? nullptr : lds + (C::PAIRS + pl) * PADN;
  LdsFft<NFFT, E, -1, false, SPLIT>::run(v, my, my_im, tw, tid);
  // Separate the two real spectra plane by plane (each output component needs one plane only):
  //   re plane: Xa.re = (Zr[k] + Zr[n-k]) / 2,  Xb.im = (Zr[n-k] - Zr[k]) / 2
  //   im plane: Xa.im = (Zi[k] - Zi[n-k]) / 2,  Xb.re = (Zi[k] + Zi[n-k]) / 2
  // Thread (pair p, bin phase kq) covers bins kq, kq + T, ...; lanes run over pairs, so the two
  // stores of a bin fill a run of FR consecutive frames of one row.
  const float hs = 0.5f * scale;
  const int p = threadIdx.x % C::PAIRS;
  const int kq = threadIdx.x / C::PAIRS;
  const int fe = f0 + 2 * p;
  const float* zp = lds + p * PADN;
  const size_t ob = (size_t)b * n_bins * n_frames + fe;
  const bool st_a = fe < n_frames, st_b = fe + 1 < n_frames;
  if constexpr (!SPLIT) {
    const float* zq = lds + (C::PAIRS + p) * PADN;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      my[lds_pad(tid + T * e)] = v[e].x;
      my_im[lds_pad(tid + T * e)] = v[e].y;
    }
    __syncthreads();
    for (int k = kq; k < n_bins; k += T) {
      const int ik = lds_pad(k), inr = lds_pad((NFFT - k) & (NFFT - 1));
      const float zr = zp[ik], yr = zp[inr], zi = zq[ik], yi = zq[inr];
      const size_t o = ob + (size_t)k * n_frames;
      if (st_a) {
        st_stream(out_re + o, (zr + yr) * hs);
        st_stream(out_im + o, (zi - yi) * hs);
      }
      if (st_b) {
        st_stream(out_re + o + 1, (zi + yi) * hs);
        st_stream(out_im + o + 1, (yr - zr) * hs);
      }
    }
    return;
  }
#pragma unroll
  for (int plane = 0; plane < 2; ++plane) {
#pragma unroll
    for (int e = 0; e < E; ++e) my[lds_pad(tid + T * e)] = plane ? v[e].y : v[e].x;
    __syncthreads();
    float* oa = plane ? out_im : out_re;  // Xa component written in this phase
    float* obp = plane ? out_re : out_im;  // Xb component written in this phase
    for (int k = kq; k < n_bins; k += T) {
      const float z = zp[lds_pad(k)];
      const float y = zp[lds_pad((NFFT - k) & (NFFT - 1))];
      const size_t o = ob + (size_t)k * n_frames;
      if (st_a) st_stream(oa + o, (plane ? z - y : z + y) * hs);
      if (st_b) st_stream(obp + o + 1, (plane ? z + y : y - z) * hs);
    }
    if (plane == 0) __syncthreads();
  }
}

template <int NFFT>
static hipError_t launch_stft_n(const StftArgs& a) {
  using C = StftCfg<NFFT>;
  const int tiles = (a.n_frames + C::FR - 1) / C::FR;
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
