// Fused STFT and inverse STFT for n_fft that is not a power of two: one Bluestein chain per frame
// (framing, padding, window and the (freq, time) layout fused in the forward kernel; completion,
// window, overlap-add and envelope in the inverse kernel).
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

template <int M, int E, int FR, bool FM = false>
__global__ __launch_bounds__((StftBlueCfg<M, E, FR>::THREADS)) void stft_blue_kernel(
    const float* __restrict__ sig, const float* __restrict__ win, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ chirp, const float2* __restrict__ hs,
    const float2* __restrict__ tw_f, const float2* __restrict__ tw_i, int n, int length, int hop, int pad,
    int n_frames, int n_bins, int tiles_per_signal, float scale) {
  using C = StftBlueCfg<M, E, FR>;
  constexpr int T = C::T, EIN = C::EIN, EH = E / 2, AREA = C::AREA, THREADS = C::THREADS;
  __shared__ __attribute__((aligned(16))) float lds[FR * AREA];
  const unsigned tile = xcd_tile_remap32(blockIdx.x, gridDim.x);  // 32-bit: grids below 2^31 (launcher)
  const unsigned b = tile / (unsigned)tiles_per_signal;
  const int f0 = (int)(tile - b * (unsigned)tiles_per_signal) * FR;
  const int tid = threadIdx.x % T;
  const int fl = threadIdx.x / T;
  const int f = f0 + fl;
  const float* x = sig + (size_t)b * length;
  // block-uniform: no padding anywhere in the tile's span (64-bit: frames past the end count)
  const long long s0 = (long long)f0 * hop - pad;
  const bool interior = s0 >= 0 && s0 + (long long)(FR - 1) * hop + n <= length;
  // the frame's loads at clamped indices and without branches, so that every element's loads
  // issue before the first wait (under a bounds test the compiler waited for each element's loads
  // before issuing the next); a slot past the frame or past the last frame is multiplied by zero
  float xs[EIN], ws[EIN];
  float2 cs[EIN];
#pragma unroll
  for (int e = 0; e < EIN; ++e) {
    const int i = tid + T * e;
    const int ic = i < n ? i : n - 1;
    int idx = f * hop + ic - pad;
    if (!interior) {
      // reflect without repeating the edge sample (torch.nn.functional.pad mode="reflect")
      idx = idx < 0 ? -idx : idx;
      idx = idx >= length ? 2 * (length - 1) - idx : idx;
      idx = idx < 0 ? 0 : (idx >= length ? length - 1 : idx);
    }
    xs[e] = x[idx];
    ws[e] = win[ic];
    cs[e] = chirp[ic];
  }
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    float2 y = make_float2(0.0f, 0.0f);
    if (e < EIN) {
      const int i = tid + T * e;
      const float m = (i < n && f < n_frames) ? 1.0f : 0.0f;
      // the reference's order: frame * window, then * chirp (real input: two products)
      const float xw = xs[e < EIN ? e : 0] * ws[e < EIN ? e : 0] * m;
      const float2 c = cs[e < EIN ? e : 0];
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
  if constexpr (FM) {
    // frames-major output (batch, n_frames, n_bins): the tile's frames are consecutive rows, one
    // contiguous run of nfr * n_bins floats per plane written by consecutive lanes
    const int nfr = n_frames - f0 < FR ? n_frames - f0 : FR;
    const size_t ob = ((size_t)b * n_frames + f0) * n_bins;
    float* cre = out_re + ob;
    float* cim = out_im + ob;
    const float rb = 1.0f / (float)n_bins;
    // lanes start early by the run's misalignment to a 128-byte line, so full-wave stores cover
    // whole lines (non-temporal stores of partial lines each reach HBM)
    const int sh = (int)((reinterpret_cast<uintptr_t>(cre) >> 2) & 31);
    for (int i = (int)threadIdx.x - sh; i < nfr * n_bins; i += THREADS) {
      if (i < 0) continue;
      int k;
      const int fl = divmod_small(i, n_bins, rb, k);
      const float2 q = reinterpret_cast<const float2*>(lds + fl * AREA)[k];
      st_stream(cre + i, q.x);
      st_stream(cim + i, q.y);
    }
    return;
  }
  constexpr int KS = THREADS / FR;  // bins per step
  const int fr = threadIdx.x % FR;
  const int kb = threadIdx.x / FR;
  if (f0 + fr >= n_frames) return;
  const float2* pb = reinterpret_cast<const float2*>(lds + fr * AREA);
  // 32-bit offsets from the signal's (uniform) base: the host keeps n_bins * n_frames below 2^30
  const size_t ob = (size_t)b * n_bins * n_frames + f0;
  float* ore = out_re + ob;
  float* oim = out_im + ob;
  unsigned off = (unsigned)(fr + kb * n_frames);
  const unsigned step = (unsigned)(KS * n_frames);
  for (int k = kb; k < n_bins; k += KS) {
    const float2 q = pb[k];
    ore[off] = q.x;
    oim[off] = q.y;
    off += step;
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
  if (a.frames_major)
    hipLaunchKernelGGL((stft_blue_kernel<M, E, FR, true>), dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream,
                       a.signal, a.window, a.out_re, a.out_im, a.chirp, a.hs, a.tw, a.tw_i, n_fft, a.length, a.hop,
                       a.pad, a.n_frames, a.n_bins, tiles, a.scale);
  else
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

// Inverse STFT of onesided spectra at n_fft that is not a power of two (trnfft/api.py:368-470:
// Hermitian completion, an inverse transform per frame -- the reference's Bluestein chain with
// its fp32 chirp of sign +1 -- real part, window, overlap-add, envelope division or raw sum,
// centre trim).  The tiling is the power-of-two inverse kernel's: a workgroup owns the output
// samples of `owned` frames and also transforms the halo = floor((n-1)/hop) frames before them.
//   1. the bins of FR consecutive frames are staged in the frames' LDS areas (lanes over frames:
//      each load reads consecutive frames of one bin row);
//   2. each frame's T threads form the completed spectrum times the chirp (X[n-k] = conj X[k];
//      the imaginary parts of bins 0 and n/2 are kept, as the reference keeps them), transform
//      forward, multiply by H/M, transform back, and keep Re(w[t] chirp[t]) * scale, t < n;
//   3. every owned sample gathers its covering frames from LDS (windowed sum, raw sum, envelope).
// M >= 2n - 1 (all n outputs of each frame are kept), so inputs and outputs are the elements
// e < E/2 of each thread.
//
// ADJ: the same tiling computes the gradient of the forward kernel above with respect to its
// padded signal (the forward plan's M and tables).  The forward map per frame is
// X[k] = chirp[k] sum_j w[j] x[j] chirp[j] conj(chirp[|k-j|]) (k < n_bins), so the adjoint takes
// u[k] = conj(chirp[k]) G[k] (k < n_bins, G the output gradient), convolves it with chirp[|s|]
// over s = -(n_bins-1) .. n-1 (the plan's adjoint filter spectrum; M >= n + n_bins - 1 holds it
// without wrap-around), keeps Re(conj(chirp[j]) v[j]) for j < n and overlap-adds it times the
// window (no envelope).  Outputs j < n then reach the elements e < EIN (n <= 2M/3).
template <int M, int E, int FR, bool ADJ = false>
struct IstftBlueCfg {
  static constexpr int T = M / E;
  static constexpr bool WL = T <= 64;
  static constexpr int AREA = stft_blue_area(M, FR);
  static constexpr int THREADS = FR * T;
  static constexpr int NW = ADJ ? stft_blue_nmax(M) : M / 2;  // longest n_fft: window floats in LDS
  static constexpr int EOUT = ADJ ? StftBlueCfg<M, E, 1>::EIN : E / 2;
  static_assert(FR * AREA * 4 + NW * 4 <= kLdsBytes, "inverse STFT frame tile exceeds LDS");
};

template <int M, int E, int FR, bool ADJ = false, bool FM = false>
__global__ __launch_bounds__((IstftBlueCfg<M, E, FR, ADJ>::THREADS)) void istft_blue_kernel(
    const float* __restrict__ sre, const float* __restrict__ sim, const float* __restrict__ win,
    float* __restrict__ out, const float2* __restrict__ chirp, const float2* __restrict__ hs,
    const float2* __restrict__ tw_f, const float2* __restrict__ tw_i, int n, int n_frames, int hop, int halo,
    int owned, int tiles_per_signal, int expected_len, int start, int write_len, int out_pitch, float scale) {
  using C = IstftBlueCfg<M, E, FR, ADJ>;
  constexpr int T = C::T, EH = E / 2, EOUT = C::EOUT, AREA = C::AREA, THREADS = C::THREADS;
  __shared__ __attribute__((aligned(16))) float lds[FR * AREA];
  __shared__ float wl[C::NW];
  const unsigned tile = xcd_tile_remap32(blockIdx.x, gridDim.x);  // 32-bit: grids below 2^31 (launcher)
  const unsigned b = tile / (unsigned)tiles_per_signal;
  const int t0 = (int)(tile - b * (unsigned)tiles_per_signal) * owned;  // first owned frame
  const int ta = t0 - halo > 0 ? t0 - halo : 0;          // first frame of the tile
  const int nf = (t0 + owned < n_frames ? t0 + owned : n_frames) - ta;  // frames in the tile (<= FR)
  const int K = n / 2 + 1;  // onesided bins

  // the window is requested first and written to LDS after the staging (a load-then-store here
  // waited out a full memory latency before the first spectrum load issued)
  constexpr int WI = (C::NW + THREADS - 1) / THREADS;
  float wv[WI];
#pragma unroll
  for (int j = 0; j < WI; ++j) {
    const int i = (int)threadIdx.x + THREADS * j;
    wv[j] = win[i < n ? i : n - 1];
  }
  // 1. stage bins: frame f's area = [re (K) | im (K)]; four loads in flight per thread
  if constexpr (FM) {
    // frames-major input (batch, n_frames, K): the tile's frames are consecutive rows, one
    // contiguous run of nf * K floats per plane (frames past nf stage zeros)
    const float* bre = sre + ((size_t)b * n_frames + ta) * K;
    const float* bim = sim + ((size_t)b * n_frames + ta) * K;
    const float rk = 1.0f / (float)K;
    for (int i0 = threadIdx.x; i0 < K * FR; i0 += 4 * THREADS) {
      float sr[4], si[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * THREADS;
        sr[u] = 0.0f;
        si[u] = 0.0f;
        if (i < K * nf) {
          sr[u] = bre[i];
          si[u] = bim[i];
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * THREADS;
        if (i < K * FR) {
          int k;
          const int f = divmod_small(i, K, rk, k);
          lds[f * AREA + k] = sr[u];
          lds[f * AREA + K + k] = si[u];
        }
      }
    }
  } else {
    const size_t sbase = (size_t)b * K * n_frames + ta;
    for (int i0 = threadIdx.x; i0 < K * FR; i0 += 4 * THREADS) {
      float sr[4], si[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * THREADS, f = i % FR, k = i / FR;
        sr[u] = 0.0f;
        si[u] = 0.0f;
        if (i < K * FR && f < nf) {
          sr[u] = sre[sbase + (size_t)k * n_frames + f];
          si[u] = sim[sbase + (size_t)k * n_frames + f];
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * THREADS, f = i % FR, k = i / FR;
        if (i < K * FR) {
          lds[f * AREA + k] = sr[u];
          lds[f * AREA + K + k] = si[u];
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < WI; ++j)
    if ((int)threadIdx.x + THREADS * j < n) wl[threadIdx.x + THREADS * j] = wv[j];
  __syncthreads();
  // 2. completed spectrum times the chirp, Bluestein chain
  const int fl = threadIdx.x / T, tid = threadIdx.x % T;
  float* my = lds + fl * AREA;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = tid + T * e;
    float2 y = make_float2(0.0f, 0.0f);
    if constexpr (ADJ) {
      if (e < EH && j < K) {  // conj(chirp[k]) G[k]
        const float2 c = chirp[j];
        y = cmul(make_float2(my[j], my[K + j]), make_float2(c.x, -c.y));
      }
    } else if (e < EH && j < n) {
      const float2 x = j < K ? make_float2(my[j], my[K + j]) : make_float2(my[n - j], -my[K + n - j]);
      y = cmul(x, chirp[j]);
    }
    v[e] = y;
  }
  // the transform reuses the frame's area
  if constexpr (C::WL) exchange_sync<true>();
  else __syncthreads();
  constexpr bool PF = blue_pf(M);
  LdsFft<M, E, -1, C::WL, false, true, PF>::run(v, my, nullptr, tw_f, tid);
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = cmul(v[e], hs[tid + T * e]);
  LdsFft<M, E, 1, C::WL, false, true, PF>::run(v, my, nullptr, tw_i, tid);
  if constexpr (!C::WL) __syncthreads();
#pragma unroll
  for (int e = 0; e < EOUT; ++e) {
    const int t = tid + T * e;
    if (t < n) {
      const float2 c = chirp[t];
      // inverse: Re(w[t] chirp[t]) / n; adjoint: Re(conj(chirp[t]) v[t])
      my[t] = (ADJ ? v[e].x * c.x + v[e].y * c.y : v[e].x * c.x - v[e].y * c.y) * scale;
    }
  }
  __syncthreads();
  // 3. owned samples [t0*hop, (t0+owned)*hop), the last tile up to the end of the signal; each
  //    gathers its covering frames t, t-1, ... (offsets s - t*hop < n)
  const int s_lo = t0 * hop;
  const long long s_end = (long long)(t0 + owned) * hop;
  const int s_hi = (t0 + owned >= n_frames || s_end > expected_len) ? expected_len : (int)s_end;
  float* dst = out + (size_t)b * out_pitch;
  const int t_end = ta + nf - 1;
  for (int s = s_lo + (int)threadIdx.x; s < s_hi; s += THREADS) {
    const int o = s - start;
    if (o < 0 || o >= write_len) continue;
    int t = (int)((unsigned)s / (unsigned)hop);
    if (t > t_end) t = t_end;
    float acc = 0.0f, raw = 0.0f, env = 0.0f;
    for (int j = s - t * hop; t >= ta && j < n; --t, j += hop) {
      const float x = lds[(t - ta) * AREA + j];
      const float w = wl[j];
      acc += x * w;
      raw += x;
      env += w * w;
    }
    dst[o] = ADJ ? acc : env > 1e-8f ? acc / env : raw;
  }
  // samples past the end of the signal up to the requested length are zero
  if (t0 + owned >= n_frames)
    for (int o = write_len + (int)threadIdx.x; o < out_pitch; o += THREADS) dst[o] = 0.0f;
}

template <int M, int E, int FR, bool ADJ>
static hipError_t launch_istft_blue_cfg(int n_fft, const IstftArgs& a) {
  using C = IstftBlueCfg<M, E, FR, ADJ>;
  const int bins = n_fft / 2 + 1;
  if (ADJ ? (n_fft + bins - 1 > M || n_fft > stft_blue_nmax(M)) : 2 * n_fft - 1 > M) return hipErrorInvalidValue;
  if (a.halo < 0 || a.hop < 1) return hipErrorInvalidValue;
  const int owned = FR - a.halo;
  if (owned < 1) return hipErrorInvalidValue;
  const int tiles = (a.n_frames + owned - 1) / owned;
  const long long blocks = a.batch * (long long)tiles;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream, a.spec_re, a.spec_im, a.window,
                       a.out, a.chirp, a.hs, a.blue_tw_f, a.blue_tw_i, n_fft, a.n_frames, a.hop, a.halo, owned, tiles,
                       (int)a.expected_len, (int)a.start, (int)a.write_len, (int)a.out_pitch, a.scale);
  };
  if (a.frames_major) go(istft_blue_kernel<M, E, FR, ADJ, true>);
  else go(istft_blue_kernel<M, E, FR, ADJ, false>);
  return hipGetLastError();
}

template <int M>
static hipError_t launch_istft_blue_m(int n_fft, const IstftArgs& a) {
  // the adjoint runs on the forward plan's tables (the forward kernel's elements per thread)
  if (a.adjoint) return launch_istft_blue_cfg<M, stft_blue_epth(M), stft_blue_adj_frames(M), true>(n_fft, a);
  return launch_istft_blue_cfg<M, istft_blue_epth(M), istft_blue_frames(M), false>(n_fft, a);
}

hipError_t launch_istft_blue(int n_fft, const IstftArgs& a) {
  switch (a.m) {
    case 32: return launch_istft_blue_m<32>(n_fft, a);
    case 64: return launch_istft_blue_m<64>(n_fft, a);
    case 96: return launch_istft_blue_m<96>(n_fft, a);
    case 128: return launch_istft_blue_m<128>(n_fft, a);
    case 192: return launch_istft_blue_m<192>(n_fft, a);
    case 256: return launch_istft_blue_m<256>(n_fft, a);
    case 384: return launch_istft_blue_m<384>(n_fft, a);
    case 512: return launch_istft_blue_m<512>(n_fft, a);
    case 768: return launch_istft_blue_m<768>(n_fft, a);
    case 1024: return launch_istft_blue_m<1024>(n_fft, a);
    case 1536: return launch_istft_blue_m<1536>(n_fft, a);
    case 2048: return launch_istft_blue_m<2048>(n_fft, a);
    case 3072: return launch_istft_blue_m<3072>(n_fft, a);
    case 4096: return launch_istft_blue_m<4096>(n_fft, a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfa
