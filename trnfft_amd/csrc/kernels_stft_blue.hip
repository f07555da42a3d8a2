// Fused STFT for n_fft that is not a power of two: framing + reflect padding + window + one
// Bluestein transform per frame + onesided slice + (freq, time) layout in one kernel.
#include "kernels.h"

namespace tfa {

// Non-power-of-two n_fft: the reference transforms every frame with its Bluestein chain
// (trnfft/api.py:339-349 -> trnfft/fft_core.py:1285-1376), whose fp32 chirp is not exactly
// Hermitian-symmetric, so two real frames cannot share a transform here; each frame gets its own
// length-M transform pair.  One workgroup takes FR consecutive frames of one signal:
//   1. the T = M/E threads of a frame load its samples (reflect padding at the signal edges),
//      window them and multiply by the chirp; samples n..M-1 are zero;
//   2. forward M-point LDS transform, times the filter spectrum H/M, inverse M-point transform;
//   3. bins k < n_bins times the chirp and the scale are staged in the frame's LDS area;
//   4. lanes run over the FR frames for each bin, so the (batch, bins, frames) rows are written
//      in runs of FR consecutive floats.
// M only has to hold the linear convolution for the kept bins: output k < n_bins sums
// y[j] h[k - j] over j < n, i.e. the filter taps -(n-1) .. n_bins-1, so with only those taps in the
// filter (the plan's) any M >= n + n_bins - 1 gives the reference's values without wrap-around,
// and M is the shortest power of two or 3 * 2^k that does (768 for n_fft = 400 onesided, against
// the reference's 1024).  The samples are the elements e < EIN of each thread and the kept bins
// (n_bins <= M/2) the elements e < E/2.
template <int M, int E, int FR>
struct StftBlueCfg {
  static constexpr int T = M / E;
  static constexpr int EIN = (stft_blue_nmax(M) + T - 1) / T < E ? (stft_blue_nmax(M) + T - 1) / T : E;
  static constexpr bool WL = T <= 64;  // transform inside one wavefront
  static constexpr int AREA = stft_blue_area(M, FR);
  static constexpr int THREADS = FR * T;
  static_assert(FR * AREA * 4 <= kLdsBytes, "STFT frame tile exceeds LDS");
  static_assert(AREA % 4 == 0, "frame areas start 16-byte aligned");
};

template <int M, int E, int FR>
__global__ __launch_bounds__((StftBlueCfg<M, E, FR>::THREADS)) void stft_blue_kernel(
    const float* __restrict__ sig, const float* __restrict__ win, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ chirp, const float2* __restrict__ hs,
    const float2* __restrict__ tw_f, const float2* __restrict__ tw_i, int n, int length, int hop, int pad,
    int n_frames, int n_bins, int tiles_per_signal, float scale) {
  using C = StftBlueCfg<M, E, FR>;
  constexpr int T = C::T, EIN = C::EIN, EH = E / 2, AREA = C::AREA, THREADS = C::THREADS;
  __shared__ __attribute__((aligned(16))) float lds[FR * AREA];
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_signal;
  const int f0 = (int)(tile % tiles_per_signal) * FR;
  const int tid = threadIdx.x % T;
  const int fl = threadIdx.x / T;
  const int f = f0 + fl;
  const float* x = sig + (size_t)b * length;
  // block-uniform: no padding anywhere in the tile's span (64-bit: frames past the end count)
  const long long s0 = (long long)f0 * hop - pad;
  const bool interior = s0 >= 0 && s0 + (long long)(FR - 1) * hop + n <= length;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid + T * e;
    float2 y = make_float2(0.0f, 0.0f);
    if (e < EIN && i < n && f < n_frames) {
      int idx = f * hop + i - pad;
      if (!interior) {
        // reflect without repeating the edge sample (torch.nn.functional.pad mode="reflect")
        idx = idx < 0 ? -idx : idx;
        idx = idx >= length ? 2 * (length - 1) - idx : idx;
        idx = idx < 0 ? 0 : (idx >= length ? length - 1 : idx);
      }
      // the reference's order: frame * window, then * chirp (real input: two products)
      const float xw = x[idx] * win[i];
      const float2 c = chirp[i];
      y = make_float2(xw * c.x, xw * c.y);
    }
    v[e] = y;
  }
  float* my = lds + fl * AREA;
  constexpr bool PF = blue_pf(M);
  LdsFft<M, E, -1, C::WL, false, true, PF>::run(v, my, nullptr, tw_f, tid);
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = cmul(v[e], hs[tid + T * e]);
  LdsFft<M, E, 1, C::WL, false, true, PF>::run(v, my, nullptr, tw_i, tid);
  // a transform spread over several wavefronts may still be reading its last exchange
  if constexpr (!C::WL) __syncthreads();
  float2* sp = reinterpret_cast<float2*>(my);
#pragma unroll
  for (int e = 0; e < EH; ++e) {
    const int k = tid + T * e;
    if (k < n_bins) {
      const float2 y = cmul(v[e], chirp[k]);
      sp[k] = make_float2(y.x * scale, y.y * scale);
    }
  }
  __syncthreads();
  constexpr int KS = THREADS / FR;  // bins per step
  const int fr = threadIdx.x % FR;
  const int kb = threadIdx.x / FR;
  if (f0 + fr >= n_frames) return;
  const float2* pb = reinterpret_cast<const float2*>(lds + fr * AREA);
  const size_t ob = (size_t)b * n_bins * n_frames + f0 + fr;
  float* ore = out_re + ob;
  float* oim = out_im + ob;
  for (int k = kb; k < n_bins; k += KS) {
    const float2 q = pb[k];
    ore[(size_t)k * n_frames] = q.x;
    oim[(size_t)k * n_frames] = q.y;
  }
}

template <int M>
static hipError_t launch_stft_blue_m(int n_fft, const StftArgs& a) {
  constexpr int E = stft_blue_epth(M);
  constexpr int FR = stft_blue_frames(M);
  using C = StftBlueCfg<M, E, FR>;
  if (n_fft + a.n_bins - 1 > M || 2 * a.n_bins > M || a.n_bins > n_fft || n_fft > stft_blue_nmax(M))
    return hipErrorInvalidValue;
  const int tiles = (a.n_frames + FR - 1) / FR;
  const long long blocks = a.batch * (long long)tiles;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((stft_blue_kernel<M, E, FR>), dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream,
                     a.signal, a.window, a.out_re, a.out_im, a.chirp, a.hs, a.tw, a.tw_i, n_fft, a.length, a.hop,
                     a.pad, a.n_frames, a.n_bins, tiles, a.scale);
  return hipGetLastError();
}

hipError_t launch_stft_blue(int n_fft, const StftArgs& a) {
  switch (a.m) {
    case 32: return launch_stft_blue_m<32>(n_fft, a);
    case 64: return launch_stft_blue_m<64>(n_fft, a);
    case 96: return launch_stft_blue_m<96>(n_fft, a);
    case 128: return launch_stft_blue_m<128>(n_fft, a);
    case 192: return launch_stft_blue_m<192>(n_fft, a);
    case 256: return launch_stft_blue_m<256>(n_fft, a);
    case 384: return launch_stft_blue_m<384>(n_fft, a);
    case 512: return launch_stft_blue_m<512>(n_fft, a);
    case 768: return launch_stft_blue_m<768>(n_fft, a);
    case 1024: return launch_stft_blue_m<1024>(n_fft, a);
    case 1536: return launch_stft_blue_m<1536>(n_fft, a);
    case 2048: return launch_stft_blue_m<2048>(n_fft, a);
    case 3072: return launch_stft_blue_m<3072>(n_fft, a);
    case 4096: return launch_stft_blue_m<4096>(n_fft, a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfa
