// Fused inverse STFT of onesided spectra: Hermitian completion, inverse transform, window,
// overlap-add, window-envelope normalisation and the centre trim in one kernel.
//
// The reference (trnfft/api.py:368-470) materialises the completed two-sided spectrum, runs a
// complex inverse per frame, keeps the real part, and then overlap-adds with index_add into an
// output, a raw (unwindowed) sum and a window-square envelope before dividing where the envelope
// exceeds 1e-8 (raw sum elsewhere).  Here one workgroup owns a run of output samples:
//   1. the bins of FR consecutive frames are staged into LDS (lanes over frames: each load
//      instruction reads consecutive frames of one bin row of the (batch, bins, frames) input,
//      the layout the forward STFT writes; or consecutive bins of the (batch, frames, bins) one);
//   2. two real frames share one complex inverse transform: Z = X_a + i X_b with X_a, X_b the
//      Hermitian completions of onesided spectra (imaginary parts of bins 0 and n/2 dropped, as
//      the reference's real part drops them), or the Hermitian parts (X[k] + conj X[n-k]) / 2 of
//      two-sided ones (the reference keeps the real part of each frame's inverse transform), so
//      IFFT(Z) = x_a + i x_b;
//   3. every output sample the workgroup owns gathers its covering frames from LDS: the windowed
//      sum, the raw sum and the envelope, then the normalised sample is written once.
// A sample is covered by frames t with t*hop <= s < t*hop + n, so a workgroup that owns the
// samples of frames [t0, t0 + FR') also transforms the H = floor((n-1)/hop) frames before t0
// (recomputed halo, no atomics and no second pass).
//
// ADJ: the same kernel computes the gradient of the forward STFT with respect to its (padded)
// signal, the adjoint of frame gather + window + onesided transform: per frame the adjoint of the
// r2c transform (a Hermitian-completed inverse transform with the interior bins halved against
// bins 0 and n/2, unscaled), times the window, overlap-added without the envelope division.
#include "kernels.h"

namespace tfa {

// MAXP caps the frame pairs per workgroup (istft_threads(NFFT) / T in the measured shape; more
// frames per workgroup cost LDS and resident workgroups without shortening the gather).
// TS: two-sided spectra (n_fft bins per frame), whose pair regions hold 4 n_fft staged floats.
template <int NFFT, int E_ = istft_epth(NFFT), int MAXP = istft_threads(NFFT) / (NFFT / E_), bool TS = false>
struct IstftCfg {
  static constexpr int E = E_;
  static constexpr int T = NFFT / E;
  static constexpr int F = TS ? NFFT : NFFT / 2 + 1;        // bins per frame
  // floats per pair region (>= 4F staged bins, >= 2n exchange and frames; a multiple of 4)
  static constexpr int RP = TS ? 4 * NFFT + 4 : 2 * lds_pad(NFFT) + 4;
  static constexpr int PAIRS_T = 1024 / T < MAXP ? 1024 / T : MAXP;
  static constexpr int PAIRS_L = (kLdsBytes - NFFT * 4) / (RP * 4);
  static constexpr int PAIRS = PAIRS_T < PAIRS_L ? PAIRS_T : PAIRS_L;
  static constexpr int FR = 2 * PAIRS;  // frames per workgroup (owned + halo)
  static constexpr int THREADS = PAIRS * T;
  static_assert(PAIRS >= 1 && RP >= 4 * F && RP >= 2 * NFFT, "istft tile");
};

template <int NFFT, int E_ = istft_epth(NFFT), int MAXP = istft_threads(NFFT) / (NFFT / E_), bool ADJ = false,
          bool FM = false, bool TS = false>
__global__ __launch_bounds__((IstftCfg<NFFT, E_, MAXP, TS>::THREADS)) void istft_kernel(
    const float* __restrict__ sre, const float* __restrict__ sim, const float* __restrict__ win,
    float* __restrict__ out, const float2* __restrict__ tw, int n_frames, int hop, int halo, int owned,
    int tiles_per_signal, long long expected_len, long long start, long long write_len, long long out_pitch,
    float scale, int vec4) {
  using C = IstftCfg<NFFT, E_, MAXP, TS>;
  static_assert(!(ADJ && TS), "the adjoint is of the onesided forward transform");
  constexpr int E = C::E, T = C::T, F = C::F, RP = C::RP, FR = C::FR, THREADS = C::THREADS;
  constexpr bool WL = T <= 64;
  // RP is a multiple of 4: every pair region and frame row is 16-byte aligned
  __shared__ __attribute__((aligned(16))) float2 lds2[C::PAIRS * RP / 2];
  __shared__ __attribute__((aligned(16))) float wl[NFFT];
  float* lds = reinterpret_cast<float*>(lds2);
  // 32-bit tile arithmetic (the launcher keeps the grid below 2^31 and the host keeps a signal's
  // bins * frames below 2^31)
  const unsigned tile = xcd_tile_remap32(blockIdx.x, gridDim.x);
  const unsigned b = tile / (unsigned)tiles_per_signal;
  const int t0 = (int)(tile - b * (unsigned)tiles_per_signal) * owned;  // first owned frame
  const int ta = t0 - halo > 0 ? t0 - halo : 0;          // first frame of the tile
  const int nf = (t0 + owned < n_frames ? t0 + owned : n_frames) - ta;  // frames in the tile (<= FR)

  // the window is requested first and written to LDS once the tile's loads are in flight (a
  // load-then-store here waited out a full memory latency before the first spectrum load issued)
  constexpr int WI = (NFFT + THREADS - 1) / THREADS;
  float wv[WI];
#pragma unroll
  for (int j = 0; j < WI; ++j) {
    const int i = (int)threadIdx.x + THREADS * j;
    wv[j] = win[i < NFFT ? i : NFFT - 1];
  }
  // 1. stage bins: region of pair p = [re_a | im_a | re_b | im_b], F floats each.  Every load of
  //    the tile is issued before the first LDS write (a load-then-store loop would wait out the
  //    full memory latency once per iteration).
  if constexpr (FM) {
    // frames-major input (batch, n_frames, F): the tile's frames are consecutive rows, one
    // contiguous run of nf * F floats per plane read by consecutive lanes
    // (32-bit byte offsets from the run's wave-uniform bases; the lane's (frame, bin) advances by
    // THREADS entries per step without a division)
    const char* bre = reinterpret_cast<const char*>(sre + ((size_t)b * n_frames + ta) * F);
    const char* bim = reinterpret_cast<const char*>(sim + ((size_t)b * n_frames + ta) * F);
    constexpr int SJ = (FR * F + THREADS - 1) / THREADS;
    const int cnt = nf * F;
    float sr[SJ], si[SJ];
#pragma unroll
    for (int it = 0; it < SJ; ++it) {
      const int i = (int)threadIdx.x + THREADS * it;
      sr[it] = 0.0f;
      si[it] = 0.0f;
      if (i < cnt) {
        const unsigned o = (unsigned)i * 4u;
        sr[it] = *reinterpret_cast<const float*>(bre + o);
        si[it] = *reinterpret_cast<const float*>(bim + o);
      }
    }
#pragma unroll
    for (int j = 0; j < WI; ++j)  // (every lane in range when the steps cover the window exactly:
                                  // no branch for the compiler to sink the window's load into)
      if (THREADS * WI == NFFT || (int)threadIdx.x + THREADS * j < NFFT) wl[threadIdx.x + THREADS * j] = wv[j];
    constexpr int DF = THREADS / F, DK = THREADS % F;
    int f = (int)threadIdx.x / F, k = (int)threadIdx.x - f * F;
#pragma unroll
    for (int it = 0; it < SJ; ++it) {
      if ((int)threadIdx.x + THREADS * it < FR * F) {
        float* r = lds + (f >> 1) * RP + (f & 1) * 2 * F;
        r[k] = sr[it];
        r[F + k] = si[it];
      }
      k += DK;
      f += DF;
      if (k >= F) {
        k -= F;
        ++f;
      }
    }
  } else {
    // (batch, F, n_frames): lane fs of every KS-lane group reads frame fs of bin rows k0,
    // k0 + KS, ... (THREADS is a multiple of FR, so a lane keeps its frame): one 32-bit offset
    // step per load from the signal's base (the former per-load 64-bit index arithmetic was a
    // quarter of the kernel's VALU work)
    constexpr int KS = THREADS / FR;
    static_assert(THREADS % FR == 0, "lanes keep their frame across the staging steps");
    const int fs = (int)threadIdx.x % FR, k0 = (int)threadIdx.x / FR;
    // 32-bit byte offsets from the signal's wave-uniform bases (one offset add per load, the base
    // in scalar registers), and no conditional loads: a lane past the tile's last frame (last tile
    // of a signal) reads that last frame and keeps zero (a frame shares its complex transform with
    // its pair partner, whose rounding a nonzero partner would change), a lane past the last bin
    // row reads the last row and writes nothing to LDS
    const char* bre = reinterpret_cast<const char*>(sre + (size_t)b * F * n_frames + ta);
    const char* bim = reinterpret_cast<const char*>(sim + (size_t)b * F * n_frames + ta);
    constexpr int SI = (F + KS - 1) / KS;
    float sr[SI], si[SI];
    {
      const bool fok = fs < nf;
      const int fsc = fok ? fs : nf - 1;
      unsigned ob = (unsigned)(fsc + k0 * n_frames) * 4u;
      const unsigned stepb = (unsigned)(KS * n_frames) * 4u;
      const unsigned lastb = (unsigned)(fsc + (F - 1) * n_frames) * 4u;
#pragma unroll
      for (int it = 0; it < SI; ++it) {
        // plain loads: a bin row segment is FR frames (64 bytes at n_fft 512), so a cache line
        // is shared with the neighbouring tile, which then finds it in L2 (measured 4 % faster)
        const unsigned o = k0 + KS * it < F ? ob : lastb;
        const float vr = *reinterpret_cast<const float*>(bre + o);
        const float vi = *reinterpret_cast<const float*>(bim + o);
        sr[it] = fok ? vr : 0.0f;
        si[it] = fok ? vi : 0.0f;
        ob += stepb;
      }
    }
#pragma unroll
    for (int j = 0; j < WI; ++j)  // (every lane in range when the steps cover the window exactly:
                                  // no branch for the compiler to sink the window's load into)
      if (THREADS * WI == NFFT || (int)threadIdx.x + THREADS * j < NFFT) wl[threadIdx.x + THREADS * j] = wv[j];
    float* sreg = lds + (fs >> 1) * RP + (fs & 1) * 2 * F + k0;
    // a lane past the last bin row writes its (clamped) values to the pair region's unused tail:
    // a store under `k < F` had the compiler sink that step's loads into the branch, one more
    // memory round trip for the workgroup
    float* spare = lds + (fs >> 1) * RP + 4 * F;
    static_assert(RP >= 4 * F + 2, "a pair region keeps two spare floats past its bins");
#pragma unroll
    for (int it = 0; it < SI; ++it) {
      const bool in = k0 + KS * it < F;
      *(in ? sreg + KS * it : spare) = sr[it];
      *(in ? sreg + F + KS * it : spare + 1) = si[it];
    }
  }
  __syncthreads();
  // 2. one complex inverse transform per frame pair
  const int pl = threadIdx.x / T, tid = threadIdx.x % T;
  float* reg = lds + pl * RP;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = tid + T * e;
    if constexpr (TS) {
      // two-sided: a frame is Re(IFFT(X)) = IFFT(H) with H[k] = (X[k] + conj X[n-k]) / 2, its
      // Hermitian part, so two frames still share one transform: Z = H_a + i H_b (the halving is
      // folded into the scale)
      const int q = (NFFT - k) & (NFFT - 1);
      const float har = reg[k] + reg[q], hai = reg[F + k] - reg[F + q];
      const float hbr = reg[2 * F + k] + reg[2 * F + q], hbi = reg[3 * F + k] - reg[3 * F + q];
      v[e] = make_float2((har - hbi) * (0.5f * scale), (hai + hbr) * (0.5f * scale));
    } else if (k <= NFFT / 2) {  // Z = X_a + i X_b
      float ra = reg[k], ia = reg[F + k], rb = reg[2 * F + k], ib = reg[3 * F + k];
      if ((e == 0 || e == E / 2) && tid == 0) {
        // bins 0 and n/2 (k = 0 and T * E / 2): their imaginary parts are dropped; the adjoint
        // counts them once against twice for the interior bins
        ia = 0.0f;
        ib = 0.0f;
        if constexpr (ADJ) {
          ra *= 2.0f;
          rb *= 2.0f;
        }
      }
      v[e] = make_float2((ra - ib) * scale, (ia + rb) * scale);
    } else {              // X[k] = conj X[n-k]:  Z = (ra + ib) + i (rb - ia) at n-k
      const int q = NFFT - k;
      v[e] = make_float2((reg[q] + reg[3 * F + q]) * scale, (reg[2 * F + q] - reg[F + q]) * scale);
    }
  }
  exchange_sync<WL>();  // the transform reuses this pair's region
  LdsFft<NFFT, E, 1, WL, false, true, istft_pf(NFFT)>::run(v, reg, nullptr, tw, tid);  // interleaved exchange
#pragma unroll
  for (int e = 0; e < E; ++e) {
    reg[tid + T * e] = v[e].x;         // frame 2p
    reg[NFFT + tid + T * e] = v[e].y;  // frame 2p + 1
  }
  __syncthreads();
  // 3. owned samples: [t0*hop, (t0+owned)*hop), the last tile up to the end of the signal.
  //    32-bit sample indices (the host bounds the signal length); one division per sample: the
  //    last covering frame, then back one hop per earlier frame while the offset stays < n.
  const int s_lo = t0 * hop;  // <= (n_frames - 1) * hop < expected_len
  const long long s_end = (long long)(t0 + owned) * hop;
  const int s_hi = (t0 + owned >= n_frames || s_end > expected_len) ? expected_len : (int)s_end;
  float* dst = out + (size_t)b * out_pitch;
  const int t_end = ta + nf - 1;
  const bool interior = halo < 4 && t0 >= halo && t0 + owned < n_frames && s_end <= expected_len;
  if (vec4 && interior && THREADS % (hop >> 2) == 0) {
    // the interior path below with four consecutive samples per thread (phase r = 4 * (thread
    // mod hop/4)): one 16-byte LDS read per covering frame and one 16-byte store per four
    // samples; hop being a multiple of 4, the four samples have the same covering frames
    const int q = hop >> 2;
    int rq;
    const int tq = divmod_small((int)threadIdx.x, q, 1.0f / (float)q, rq);
    const int r = 4 * rq;
    const int tstep = THREADS / q;
    const int nc = (NFFT - 1 - r) / hop + 1;
    float4 wv[4];
    float4 env = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      wv[m] = m < nc ? *reinterpret_cast<const float4*>(wl + r + m * hop) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (m < nc) {
        env.x += wv[m].x * wv[m].x;
        env.y += wv[m].y * wv[m].y;
        env.z += wv[m].z * wv[m].z;
        env.w += wv[m].w * wv[m].w;
      }
    }
    const float4 inv = make_float4(1.0f / env.x, 1.0f / env.y, 1.0f / env.z, 1.0f / env.w);
    for (int t = t0 + tq; t < t0 + owned; t += tstep) {
      const int o = t * hop + r - (int)start;
      if (o < 0 || o >= write_len) continue;
      float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f), raw = acc;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m < nc) {
          const int f = t - m - ta;
          const float4 x = *reinterpret_cast<const float4*>(lds + (f >> 1) * RP + (f & 1) * NFFT + r + m * hop);
          acc.x += x.x * wv[m].x;
          acc.y += x.y * wv[m].y;
          acc.z += x.z * wv[m].z;
          acc.w += x.w * wv[m].w;
          raw.x += x.x;
          raw.y += x.y;
          raw.z += x.z;
          raw.w += x.w;
        }
      }
      float4 y = acc;
      if constexpr (!ADJ) {
        y.x = env.x > 1e-8f ? acc.x * inv.x : raw.x;
        y.y = env.y > 1e-8f ? acc.y * inv.y : raw.y;
        y.z = env.z > 1e-8f ? acc.z * inv.z : raw.z;
        y.w = env.w > 1e-8f ? acc.w * inv.w : raw.w;
      }
      st_stream4(dst + o, y);
    }
    return;  // not the last tile: no zero fill
  }
  if (THREADS % hop == 0 && interior) {
    // interior tile (every owned sample has all its covering frames in the tile) and a hop that
    // divides the thread count: each thread keeps one phase r = s mod hop, so its covering frames
    // t, t-1, ... meet it at the fixed offsets r, r + hop, ... of their windows; the window
    // values and the envelope (summed in the same order as below) are computed once per thread
    // and the envelope division becomes one reciprocal per thread
    const int r = (int)threadIdx.x % hop;
    const int tstep = THREADS / hop;
    const int nc = (NFFT - 1 - r) / hop + 1;  // covering frames of phase r (<= halo + 1 <= 4)
    float wv[4], env = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      wv[m] = m < nc ? wl[r + m * hop] : 0.0f;
      if (m < nc) env += wv[m] * wv[m];
    }
    const bool norm = env > 1e-8f;
    const float inv = 1.0f / env;
    for (int t = t0 + (int)threadIdx.x / hop; t < t0 + owned; t += tstep) {
      const int o = t * hop + r - (int)start;
      if (o < 0 || o >= write_len) continue;
      float acc = 0.0f, raw = 0.0f;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m < nc) {
          const int f = t - m - ta;
          const float x = lds[(f >> 1) * RP + (f & 1) * NFFT + r + m * hop];
          acc += x * wv[m];
          raw += x;
        }
      }
      st_stream(dst + o, ADJ ? acc : norm ? acc * inv : raw);  // non-temporal: whole output rows (C2 inverse 41.5 -> 38.6 us)
    }
    return;  // not the last tile: no zero fill
  }
  for (int s = s_lo + (int)threadIdx.x; s < s_hi; s += THREADS) {
    const int o = s - start;
    if (o < 0 || o >= write_len) continue;
    int t = (int)((unsigned)s / (unsigned)hop);
    if (t > t_end) t = t_end;
    float acc = 0.0f, raw = 0.0f, env = 0.0f;
    for (int j = s - t * hop; t >= ta && j < NFFT; --t, j += hop) {
      const int f = t - ta;
      const float x = lds[(f >> 1) * RP + (f & 1) * NFFT + j];
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

template <int NFFT, int MAXP, bool TS>
static hipError_t launch_istft_cfg(const IstftArgs& a) {
  using C = IstftCfg<NFFT, istft_epth(NFFT), MAXP, TS>;
  const int owned = C::FR - a.halo;
  if (owned < 1) return hipErrorInvalidValue;
  const int tiles = (a.n_frames + owned - 1) / owned;
  const long long blocks = a.batch * (long long)tiles;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream, a.spec_re, a.spec_im, a.window,
                       a.out, a.tw, a.n_frames, a.hop, a.halo, owned, tiles, (int)a.expected_len, (int)a.start,
                       (int)a.write_len, (int)a.out_pitch, a.scale, (int)a.vec4);
  };
  constexpr int E = istft_epth(NFFT);
  if constexpr (TS) {
    if (a.adjoint) return hipErrorInvalidValue;  // the adjoint is of the onesided forward transform
    if (a.frames_major) go(istft_kernel<NFFT, E, MAXP, false, true, true>);
    else go(istft_kernel<NFFT, E, MAXP, false, false, true>);
  } else if (a.adjoint) {
    if (a.frames_major) go(istft_kernel<NFFT, E, MAXP, true, true>);
    else go(istft_kernel<NFFT, E, MAXP, true, false>);
  } else {
    if (a.frames_major) go(istft_kernel<NFFT, E, MAXP, false, true>);
    else go(istft_kernel<NFFT, E, MAXP, false, false>);
  }
  return hipGetLastError();
}

// The measured shape, unless the hop is so short that the recomputed halo frames would be half
// its tile or more: then the widest tile (1024 threads, as LDS allows), same elements per thread.
template <int NFFT, bool TS>
static hipError_t launch_istft_ts(const IstftArgs& a) {
  constexpr int T = NFFT / istft_epth(NFFT);
  constexpr int FAST = istft_threads(NFFT) / T, WIDE = 1024 / T;
  if (2 * a.halo <= IstftCfg<NFFT, istft_epth(NFFT), FAST, TS>::FR) return launch_istft_cfg<NFFT, FAST, TS>(a);
  return launch_istft_cfg<NFFT, WIDE, TS>(a);
}

template <int NFFT>
static hipError_t launch_istft_n(const IstftArgs& a) {
  return a.two_sided ? launch_istft_ts<NFFT, true>(a) : launch_istft_ts<NFFT, false>(a);
}

// frames per tile of the widest shape: the hop bound the plan checks
template <int NFFT>
constexpr int istft_wide_fr(bool two_sided) {
  constexpr int W = 1024 / (NFFT / istft_epth(NFFT));
  return two_sided ? IstftCfg<NFFT, istft_epth(NFFT), W, true>::FR : IstftCfg<NFFT, istft_epth(NFFT), W>::FR;
}

int istft_frames_per_tile(int n_fft, bool two_sided) {
  switch (n_fft) {
    case 16: return istft_wide_fr<16>(two_sided);
    case 32: return istft_wide_fr<32>(two_sided);
    case 64: return istft_wide_fr<64>(two_sided);
    case 128: return istft_wide_fr<128>(two_sided);
    case 256: return istft_wide_fr<256>(two_sided);
    case 512: return istft_wide_fr<512>(two_sided);
    case 1024: return istft_wide_fr<1024>(two_sided);
    case 2048: return istft_wide_fr<2048>(two_sided);
    case 4096: return istft_wide_fr<4096>(two_sided);
    default: return 0;
  }
}

hipError_t launch_istft(int n_fft, const IstftArgs& a) {
  switch (n_fft) {
    case 16: return launch_istft_n<16>(a);
    case 32: return launch_istft_n<32>(a);
    case 64: return launch_istft_n<64>(a);
    case 128: return launch_istft_n<128>(a);
    case 256: return launch_istft_n<256>(a);
    case 512: return launch_istft_n<512>(a);
    case 1024: return launch_istft_n<1024>(a);
    case 2048: return launch_istft_n<2048>(a);
    case 4096: return launch_istft_n<4096>(a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfa
