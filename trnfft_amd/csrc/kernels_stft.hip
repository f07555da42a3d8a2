// Fused STFT: framing + reflect padding + window + FFT + onesided slice + (freq, time) layout in
// one kernel that reads the raw waveform (trnfft/api.py:291-365 materialises the padded signal,
// the frame matrix, the windowed frames and a zero imaginary plane before its per-frame c2c).
//
// The frames are real, so two of them share one complex transform: z = w*x_a + i*w*x_b gives
// X_a[k] = (Z[k] + conj(Z[n-k])) / 2 and X_b[k] = (Z[k] - conj(Z[n-k])) / (2i).
// One workgroup takes FR consecutive frames of one signal (FR/2 complex LDS transforms):
//   1. the threads of each frame pair load the pair's two frames straight from the waveform
//      (coalesced runs of consecutive samples, reflect padding at the signal edges) and window them;
//      the half-hop overlap between neighbouring frames is served by L2;
//   2. each pair is transformed (LDS Stockham; one wavefront per pair at n_fft = 512);
//   3. each pair stores its spectrum as packed entries (Z[k], Z[n-k]), k <= n/2, one float4 each;
//      frames-major output (batch, frames, bins) -- the memory order of torch.stft's result and
//      of trnfft's transposed view -- is then one contiguous run per plane for the whole tile;
//      for (batch, bins, frames) lanes run over consecutive frames and read one entry per output
//      bin, so every store instruction writes FR contiguous floats of bin rows.
// The window is pre-scaled by scale/2 (the 1/2 of the pair separation, and the normalisation), so
// the separation is two additions per output value.
#include "kernels.h"

namespace tfa {

// Frame pairs per workgroup: 8192 / n_fft (1024 threads from n_fft = 256 up), between 2 and 32.
template <int NFFT>
constexpr int stft_pairs() {
  constexpr int p = 8192 / NFFT;
  return p < 2 ? 2 : p > 32 ? 32 : p;
}
// Floats of LDS per frame pair: the interleaved exchange area of the transform, which also holds
// the packed spectrum (4 * (n/2 + 1) floats) afterwards; a multiple of 4 floats (float4 entries)
// that is 4 more than a multiple of 64, so the pair regions start on successive bank quads.
constexpr int stft_area(int n) {
  int a = (2 * (lds_pad(n) + 1) + 3) / 4 * 4;
  while (a % 64 != 4) a += 4;
  return a;
}

template <int NFFT, int PAIRS_ = stft_pairs<NFFT>(), int E_ = stft_epth(NFFT)>
struct StftCfg {
  static constexpr int E = E_;
  static constexpr int T = NFFT / E;  // threads per frame pair
  static constexpr int PAIRS = PAIRS_;
  static constexpr int FR = 2 * PAIRS;  // frames per workgroup
  static constexpr int THREADS = PAIRS * T;
  static constexpr int AREA = stft_area(NFFT);
  static constexpr int NB1 = NFFT / 2 + 1;  // onesided bins = packed entries per pair
  static_assert(PAIRS * AREA * 4 <= kLdsBytes, "STFT tile exceeds LDS");
  static_assert(THREADS % FR == 0, "the output stage maps lanes to (bin, frame)");
};

// FM: frames-major output, (batch, n_frames, n_bins): the tile's frames are consecutive rows, so
// every plane receives one contiguous run of (frames in the tile) * n_bins floats, written by
// consecutive lanes; otherwise (batch, n_bins, n_frames), FR floats per bin row.  LDNT / STNT:
// non-temporal waveform loads / frames-major stores.
template <int NFFT, bool FM = false, int PAIRS_ = stft_pairs<NFFT>(), int E_ = stft_epth(NFFT), bool LDNT = true,
          bool STNT = true, bool ALIGN = false, int OU = 0>
__global__ __launch_bounds__((StftCfg<NFFT, PAIRS_, E_>::THREADS)) void stft_kernel(
    const float* __restrict__ sig, const float* __restrict__ win, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, int length, int hop, int pad,
    int n_frames, int n_bins, int tiles_per_signal, float hs) {
  using C = StftCfg<NFFT, PAIRS_, E_>;
  constexpr int E = C::E, T = C::T, FR = C::FR, AREA = C::AREA, THREADS = C::THREADS, NB1 = C::NB1;
  __shared__ __attribute__((aligned(16))) float lds[C::PAIRS * AREA];
  const unsigned tile = xcd_tile_remap32(blockIdx.x, gridDim.x);  // 32-bit: grids below 2^31 (launcher)
  const unsigned b = tile / (unsigned)tiles_per_signal;
  const int f0 = (int)(tile - b * (unsigned)tiles_per_signal) * FR;
  const int tid = threadIdx.x % T;
  const int pl = threadIdx.x / T;
  const int fa = f0 + 2 * pl;  // frames fa (real part) and fa + 1 (imaginary part)
  const float* x = sig + (size_t)b * length;
  const int start = f0 * hop - pad;  // padded-signal origin of the tile's first frame
  const long long span = (long long)(FR - 1) * hop + NFFT;  // (frames past the end count)
  float wv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) wv[e] = win[tid + T * e] * hs;
  float2 v[E];
  if (start >= 0 && (long long)start + span <= length) {  // block-uniform: no padding inside the tile
    const float* p0 = x + (start + 2 * pl * hop) + tid;
    const float* p1 = p0 + hop;
    float a[E], c[E];
#pragma unroll
    for (int e = 0; e < E; ++e) a[e] = LDNT ? ld_stream(p0 + T * e) : p0[T * e];
#pragma unroll
    for (int e = 0; e < E; ++e) c[e] = LDNT ? ld_stream(p1 + T * e) : p1[T * e];
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = make_float2(a[e] * wv[e], c[e] * wv[e]);
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int j = tid + T * e;
      float s[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // frames past the end (never stored) read the last frame's samples
        const int fi = fa + h < n_frames ? fa + h : n_frames - 1;
        int idx = fi * hop + j - pad;
        // reflect without repeating the edge sample (torch.nn.functional.pad mode="reflect")
        idx = idx < 0 ? -idx : idx;
        idx = idx >= length ? 2 * (length - 1) - idx : idx;
        idx = idx < 0 ? 0 : (idx >= length ? length - 1 : idx);
        s[h] = x[idx] * wv[e];
      }
      v[e] = make_float2(s[0], s[1]);
    }
  }
  float* my = lds + pl * AREA;
  LdsFft<NFFT, E, -1, (T <= 64), false, true, stft_pf(NFFT)>::run(v, my, nullptr, tw, tid);
  // a transform spread over several wavefronts may still be reading its last exchange
  if constexpr (T > 64) __syncthreads();
  // packed spectrum: entry k (0..n/2) = (Z[k], Z[n-k mod n]) as one float4
  float2* sp = reinterpret_cast<float2*>(my);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = tid + T * e;
    if (e < E / 2) sp[2 * k] = v[e];              // k < n/2: first half of entry k
    else sp[2 * (NFFT - k) + 1] = v[e];           // k >= n/2: second half of entry n - k
  }
  if (tid == 0) {
    sp[1] = v[0];                  // entry 0: Z[n - 0 mod n] = Z[0]
    sp[2 * (NFFT / 2)] = v[E / 2]; // entry n/2: Z[n/2] in both halves
  }
  __syncthreads();
  if constexpr (FM) {
    const int nfr = n_frames - f0 < FR ? n_frames - f0 : FR;
    const size_t ob = ((size_t)b * n_frames + f0) * n_bins;
    float* cre = out_re + ob;
    float* cim = out_im + ob;
    // lanes start one cache line early by the run's misalignment, so every store instruction of a
    // full wave covers whole 128-byte lines (non-temporal stores of partial lines each reach HBM)
    const int sh = ALIGN ? (int)((reinterpret_cast<uintptr_t>(cre) >> 2) & 31) : 0;
    if (OU > 0 && n_bins == NB1) {
      // OU store steps at a time: their LDS entries are read together (indices clamped into the
      // tile, so the reads need no branch), then the in-range lanes store; 32-bit byte offsets
      // from the tile's (wave-uniform) run bases
      const int cnt = nfr * NB1;
      char* bre = reinterpret_cast<char*>(cre);
      char* bim = reinterpret_cast<char*>(cim);
      for (int i0 = (int)threadIdx.x - sh; i0 < cnt; i0 += OU * THREADS) {
        float4 q[OU > 0 ? OU : 1];
        bool odd[OU > 0 ? OU : 1];
#pragma unroll
        for (int u = 0; u < OU; ++u) {
          const int i = i0 + u * THREADS;
          const int ic = i < 0 ? 0 : (i < FR * NB1 ? i : FR * NB1 - 1);
          const int fl = ic / NB1, k = ic - fl * NB1;
          q[u] = reinterpret_cast<const float4*>(lds + (fl >> 1) * AREA)[k];  // (Z[k], Z[n-k])
          odd[u] = fl & 1;
        }
#pragma unroll
        for (int u = 0; u < OU; ++u) {
          const int i = i0 + u * THREADS;
          if (i >= 0 && i < cnt) {
            const float re = odd[u] ? (q[u].y + q[u].w) : (q[u].x + q[u].z);
            const float im = odd[u] ? (q[u].z - q[u].x) : (q[u].y - q[u].w);
            const unsigned o = (unsigned)i * 4u;
            st_stream(reinterpret_cast<float*>(bre + o), re);
            st_stream(reinterpret_cast<float*>(bim + o), im);
          }
        }
      }
    } else if (n_bins == NB1) {
      for (int i = (int)threadIdx.x - sh; i < nfr * NB1; i += THREADS) {
        if (i < 0) continue;
        const int fl = i / NB1, k = i - fl * NB1;
        const float4 q = reinterpret_cast<const float4*>(lds + (fl >> 1) * AREA)[k];  // (Z[k], Z[n-k])
        const bool odd = fl & 1;
        const float re = odd ? (q.y + q.w) : (q.x + q.z), im = odd ? (q.z - q.x) : (q.y - q.w);
        if constexpr (STNT) {
          st_stream(cre + i, re);
          st_stream(cim + i, im);
        } else {
          cre[i] = re;
          cim[i] = im;
        }
      }
    } else {
      // two-sided: bins above n/2 read entry n - k with its halves swapped
      for (int i = (int)threadIdx.x - sh; i < nfr * NFFT; i += THREADS) {
        if (i < 0) continue;
        const int fl = i / NFFT, k = i % NFFT;
        const bool hi = k > NFFT / 2;
        const float4 q = reinterpret_cast<const float4*>(lds + (fl >> 1) * AREA)[hi ? NFFT - k : k];
        const float zr = hi ? q.z : q.x, zi = hi ? q.w : q.y, yr = hi ? q.x : q.z, yi = hi ? q.y : q.w;
        const bool odd = fl & 1;
        st_stream(cre + i, odd ? (zi + yi) : (zr + yr));
        st_stream(cim + i, odd ? (yr - zr) : (zi - yi));
      }
    }
    return;
  }
  // lanes over consecutive frames fr: frame fr = 2p (+1) is the real (imaginary) part of pair p
  constexpr int KS = THREADS / FR;  // bins per step
  const int fr = threadIdx.x % FR;
  const int kb = threadIdx.x / FR;
  if (f0 + fr >= n_frames) return;
  const float* pbase = lds + (fr >> 1) * AREA;
  const bool odd = fr & 1;
  const size_t ob = (size_t)b * n_bins * n_frames + f0;
  // byte offsets from the wave-uniform row bases (scalar base + 32-bit vector offset stores)
  char* bre = reinterpret_cast<char*>(out_re + ob);
  char* bim = reinterpret_cast<char*>(out_im + ob);
  if (n_bins == NB1) {
    const float4* e4 = reinterpret_cast<const float4*>(pbase) + kb;
    unsigned off = (unsigned)(fr + kb * n_frames) * 4u;
    const unsigned step = (unsigned)(KS * n_frames) * 4u;
#pragma unroll
    for (int i = 0; i < (NB1 + KS - 1) / KS; ++i) {
      if (kb + KS * i < NB1) {
        const float4 q = e4[KS * i];  // (zr, zi, yr, yi) = (Z[k], Z[n-k])
        const float re = odd ? (q.y + q.w) : (q.x + q.z);
        const float im = odd ? (q.z - q.x) : (q.y - q.w);
        *reinterpret_cast<float*>(bre + off) = re;
        *reinterpret_cast<float*>(bim + off) = im;
      }
      off += step;
    }
  } else {
    // two-sided: bins above n/2 read entry n - k with its halves swapped
    for (int k = kb; k < n_bins; k += KS) {
      const bool hi = k > NFFT / 2;
      const float4 q = reinterpret_cast<const float4*>(pbase)[hi ? NFFT - k : k];
      const float zr = hi ? q.z : q.x, zi = hi ? q.w : q.y, yr = hi ? q.x : q.z, yi = hi ? q.y : q.w;
      const float re = odd ? (zi + yi) : (zr + yr);
      const float im = odd ? (yr - zr) : (zi - yi);
      const unsigned o = (unsigned)(fr + k * n_frames) * 4u;
      *reinterpret_cast<float*>(bre + o) = re;
      *reinterpret_cast<float*>(bim + o) = im;
    }
  }
}

// Frame pairs per workgroup of the frames-major kernel, from a sweep on MI355X (64 x 160000
// samples, hop n/2, 1..32 pairs): 256 threads up to n_fft = 512, 512 above (64: 30.5 us, 128:
// 31.3, 256: 32.0, 512: 32.8 against 36.8 with the bins-major tile shape, 1024: 36.2, 2048: 36.9,
// 4096: 38.9), with temporal waveform loads (the half-hop overlap of neighbouring frames then hits
// in the cache: 512 with 4 pairs 34.3 -> 32.7 us) and line-aligned non-temporal stores (256:
// 32.1 -> 29.6 us, 512: 33.0 -> 30.7-31.0, 1024: 36.2 -> 34.5; the unaligned runs wrote 1.10x
// their bytes); the onesided store loop takes three steps at a time (128: 28.5 -> 28.2 us, 512:
// 30.8 -> 30.3-30.5, 2048: 36.6 -> 36.0, 4096: 40.0 -> 38.1).  Four elements per thread (512:
// 40.5 us) or sixteen (35.5; 1024: 33.9 against 34.9, the only size where it won) were slower.
template <int NFFT>
constexpr int stft_fm_pairs() {
  constexpr int p = (NFFT <= 512 ? 256 : 512) / (NFFT / stft_epth(NFFT));
  return p < 1 ? 1 : p > 32 ? 32 : p;
}

template <int NFFT>
static hipError_t launch_stft_n(const StftArgs& a) {
  if (a.frames_major) {
    constexpr int P = stft_fm_pairs<NFFT>();
    using C = StftCfg<NFFT, P>;
    const int tiles = (a.n_frames + C::FR - 1) / C::FR;
    const long long blocks = a.batch * (long long)tiles;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL((stft_kernel<NFFT, true, P, stft_epth(NFFT), false, true, true, 3>), dim3((unsigned)blocks),
                       dim3(C::THREADS), 0, a.stream, a.signal, a.window, a.out_re, a.out_im, a.tw, a.length, a.hop,
                       a.pad, a.n_frames, a.n_bins, tiles, 0.5f * a.scale);
    return hipGetLastError();
  }
  using C = StftCfg<NFFT>;
  const int tiles = (a.n_frames + C::FR - 1) / C::FR;
  const long long blocks = a.batch * (long long)tiles;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  // stft_lds_extra: unused dynamic LDS that holds the workgroups resident per CU to one where that
  // measured faster
  hipLaunchKernelGGL((stft_kernel<NFFT>), dim3((unsigned)blocks), dim3(C::THREADS), stft_lds_extra(NFFT), a.stream,
                     a.signal, a.window, a.out_re, a.out_im, a.tw, a.length, a.hop, a.pad, a.n_frames, a.n_bins,
                     tiles, 0.5f * a.scale);
  return hipGetLastError();
}

hipError_t launch_stft(int n_fft, const StftArgs& a) {
  if (a.m != 0) return launch_stft_blue(n_fft, a);
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
