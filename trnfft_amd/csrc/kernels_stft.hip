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
//      for (batch, bins, frames) -- the reference's result layout (its ComplexTensor makes the
//      transposed planes contiguous, trnfft/complex.py:29-33) -- lanes run over consecutive frames
//      and read one entry per output bin, so every store instruction writes FR contiguous floats
//      of bin rows (stft_binrows_kernel below writes this layout as whole lines where it applies);
//      frames-major output (batch, frames, bins) -- the memory order of torch.stft's result, an
//      opt-in here -- is one contiguous run per plane for the whole tile.
// The window is pre-scaled by scale/2 (the 1/2 of the pair separation, and the normalisation), so
// the separation is two additions per output value.
#include <algorithm>
#include <cmath>

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
  // the window times hs is formed after the samples' loads are issued (formed first, the window
  // loads were waited for before the first sample load)
  float wr[E];
#pragma unroll
  for (int e = 0; e < E; ++e) wr[e] = win[tid + T * e];
  float2 v[E];
  float a[E], c[E];
  if (start >= 0 && (long long)start + span <= length) {  // block-uniform: no padding inside the tile
    const float* p0 = x + (start + 2 * pl * hop) + tid;
    const float* p1 = p0 + hop;
#pragma unroll
    for (int e = 0; e < E; ++e) a[e] = LDNT ? ld_stream(p0 + T * e) : p0[T * e];
#pragma unroll
    for (int e = 0; e < E; ++e) c[e] = LDNT ? ld_stream(p1 + T * e) : p1[T * e];
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int j = tid + T * e;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // frames past the end (never stored) read the last frame's samples
        const int fi = fa + h < n_frames ? fa + h : n_frames - 1;
        int idx = fi * hop + j - pad;
        // reflect without repeating the edge sample (torch.nn.functional.pad mode="reflect")
        idx = idx < 0 ? -idx : idx;
        idx = idx >= length ? 2 * (length - 1) - idx : idx;
        idx = idx < 0 ? 0 : (idx >= length ? length - 1 : idx);
        (h ? c : a)[e] = x[idx];
      }
    }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float wv = wr[e] * hs;
    v[e] = make_float2(a[e] * wv, c[e] * wv);
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

// ---------------------------------------------------------------------------------------------
// Bins-major spectra (batch, n_bins, n_frames) -- the reference's result layout -- as whole
// 128-byte lines.  A bin row of n_frames floats starts anywhere in a line, so spectra of fixed
// frame tiles cover the lines of every row partially; partial lines must then merge in L2 (plain
// stores), which measured 37.5 us at C2 against 28 us for whole lines stored non-temporally.
// Here each workgroup owns a contiguous frame range [R0, R1) of one signal and walks it in
// sub-tiles of 32 frames, and writes per bin row only the lines its frames complete:
//  * 8 transform waves load the sub-tile's frames (two per complex transform, as stft_kernel)
//    one sub-tile ahead, transform two pairs each in lockstep (LdsFftMulti) and leave packed
//    spectra in one of two LDS buffers;
//  * 8 store waves write the previous sub-tile's lines meanwhile: 16 lanes per line, two frames
//    per lane (one packed LDS entry, one float2 store); the frames of a line that belong to the
//    next sub-tile stay in the lanes' registers until then (the "carry").
// The roles never share a wavefront, so a transform wave's loads never wait behind stores (one
// vmcnt counter per wave counts both).  Even ranges walk forward and odd ranges backward, so
// the two partial lines at a boundary between ranges -- and the line shared by the end of bin
// row k and the start of row k + 1 (first steps of the signal's last and first ranges) -- are
// written by neighbouring workgroups in the same step, and the tile order keeps a signal's
// ranges on one XCD: they merge in its L2.
// Preconditions (host-checked): onesided, n_frames even (pairs of frames never straddle a line
// or range boundary, ranges start on even frames), output planes 8-byte aligned at the same
// offset modulo 128 bytes, length >= n_fft, (n_fft/2 + 1) * n_frames * 4 < 2^32.
template <int NFFT>
struct BinRowsCfg {
  static constexpr int E = 8, T = NFFT / E;
  static constexpr int PAIRS = 16, FR = 2 * PAIRS;        // frame pairs / frames per sub-tile
  static constexpr int TWAVES = 8, SWAVES = 8, THREADS = 64 * (TWAVES + SWAVES);
  static constexpr int PPW = 64 / T;                       // pairs a transform wave holds at once
  static constexpr int ROUNDS = PAIRS / (TWAVES * PPW);    // transforms per thread per sub-tile
  static constexpr int AREA = stft_area(NFFT), NB1 = NFFT / 2 + 1;
  static constexpr int BUF = PAIRS * AREA;                 // floats per spectra buffer
  static constexpr LdsShape S = make_shape(NFFT, E);
  static constexpr int TW = S.twoff[S.npass] + 2;          // twiddle table entries (float2)
  static constexpr int LPP = SWAVES * 4;                   // lines per store pass
  static constexpr int PASSES = (NB1 + LPP - 1) / LPP;
  static_assert(T <= 64 && 64 % T == 0 && ROUNDS >= 1 && PAIRS % (TWAVES * PPW) == 0, "pair transforms");
  static_assert(FR == 32, "a sub-tile spans one line of every bin row");
  static_assert((2 * BUF + 2 * TW + NB1) * 4 <= kLdsBytes, "STFT bin-row tile exceeds LDS");
};

// first frame of range r of q (even), r = q: n_frames
__device__ __forceinline__ int binrows_range_start(int r, int q, int n_frames) {
  return r >= q ? n_frames : (int)(((long long)n_frames * r / q) & ~1LL);
}

template <int NFFT>
__global__ __launch_bounds__(BinRowsCfg<NFFT>::THREADS) void stft_binrows_kernel(
    const float* __restrict__ sig, const float* __restrict__ win, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, int length, int hop, int pad, int n_frames,
    int q_ranges, unsigned base_mod, float hs) {
  using C = BinRowsCfg<NFFT>;
  constexpr int E = C::E, T = C::T, FR = C::FR, AREA = C::AREA, BUF = C::BUF, TW = C::TW, NB1 = C::NB1;
  constexpr int TWAVES = C::TWAVES, PPW = C::PPW, ROUNDS = C::ROUNDS, LPP = C::LPP, PASSES = C::PASSES;
  __shared__ __attribute__((aligned(16))) float lds[2 * BUF + 2 * TW + NB1];
  float2* ltw = reinterpret_cast<float2*>(lds + 2 * BUF);  // twiddles: the transforms issue no global loads
  int* o_tab = reinterpret_cast<int*>(lds + 2 * BUF + 2 * TW);  // per bin row: first frame's float within its line
  const unsigned tile = xcd_tile_remap32(blockIdx.x, gridDim.x);  // 32-bit: grids below 2^31 (launcher)
  const unsigned b = tile / (unsigned)q_ranges;
  const int r = (int)(tile - b * (unsigned)q_ranges);
  const int R0 = binrows_range_start(r, q_ranges, n_frames), R1 = binrows_range_start(r + 1, q_ranges, n_frames);
  const bool fwd = (r & 1) == 0;
  const int steps = (R1 - R0 + FR - 1) / FR;
  {
    const unsigned nfr_mod = (unsigned)n_frames & 31u;
    const unsigned rowbase_mod = base_mod + ((b * (unsigned)NB1) & 31u) * nfr_mod;
    for (int i = threadIdx.x; i < TW; i += C::THREADS) ltw[i] = tw[i];
    for (int k = threadIdx.x; k < NB1; k += C::THREADS) o_tab[k] = (int)((rowbase_mod + (unsigned)k * nfr_mod) & 31u);
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6;
  if (wave < TWAVES) {
    // ---- transform waves: pair p = (u * TWAVES + wave) * PPW + lane / T of sub-tile A holds
    // frames A + 2p (real part) and A + 2p + 1 (imaginary part)
    const int tid = threadIdx.x % T;
    const int pw = (threadIdx.x & 63) / T;
    const float* x = sig + (size_t)b * length;
    float wv[E];
#pragma unroll
    for (int e = 0; e < E; ++e) wv[e] = win[tid + T * e] * hs;
    auto sub_start = [&](int i) { return fwd ? R0 + FR * i : R1 - FR * (i + 1); };
    auto frame_start = [&](int f) {  // padded-signal position of frame f's first sample
      f = f < 0 ? 0 : (f >= n_frames ? n_frames - 1 : f);
      return f * hop - pad;
    };
    // one sub-tile's samples, read from windows clamped into the signal (frames whose window
    // leaves it are reloaded with reflection before their transform)
    auto load = [&](int A, float (&ya)[ROUNDS][E], float (&yb)[ROUNDS][E]) {
#pragma unroll
      for (int u = 0; u < ROUNDS; ++u) {
        const int p = (u * TWAVES + wave) * PPW + pw;
        int s0 = frame_start(A + 2 * p), s1 = frame_start(A + 2 * p + 1);
        s0 = s0 < 0 ? 0 : (s0 > length - NFFT ? length - NFFT : s0);
        s1 = s1 < 0 ? 0 : (s1 > length - NFFT ? length - NFFT : s1);
        const float* p0 = x + s0 + tid;
        const float* p1 = x + s1 + tid;
#pragma unroll
        for (int e = 0; e < E; ++e) ya[u][e] = p0[T * e];
#pragma unroll
        for (int e = 0; e < E; ++e) yb[u][e] = p1[T * e];
      }
    };
    float xa[ROUNDS][E], xb[ROUNDS][E];
    load(sub_start(0), xa, xb);
    for (int i = 0; i < steps; ++i) {
      const int A = sub_start(i);
      float ya[ROUNDS][E], yb[ROUNDS][E];
      // the next sub-tile (past the range's end: clamped frames, never stored; unconditional so
      // that the waits below count these loads as the youngest)
      load(sub_start(i + 1), ya, yb);
      float* buf = lds + (i & 1) * BUF;
      float2 v[ROUNDS][E];
      float* area[ROUNDS];
#pragma unroll
      for (int u = 0; u < ROUNDS; ++u) {
        const int p = (u * TWAVES + wave) * PPW + pw;
        area[u] = buf + p * AREA;
        const int s0 = frame_start(A + 2 * p), s1 = frame_start(A + 2 * p + 1);
        if (__any(s0 < 0 || s1 < 0 || s0 > length - NFFT || s1 > length - NFFT)) {
          // reflect padding (torch.nn.functional.pad mode="reflect": the edge sample is not
          // repeated); wait for these loads inside the branch, so that the common path below
          // waits only for this sub-tile's prefetched samples
#pragma unroll
          for (int e = 0; e < E; ++e) {
            int i0 = s0 + tid + T * e, i1 = s1 + tid + T * e;
            i0 = i0 < 0 ? -i0 : i0;
            i0 = i0 >= length ? 2 * (length - 1) - i0 : i0;
            i0 = i0 < 0 ? 0 : (i0 >= length ? length - 1 : i0);
            i1 = i1 < 0 ? -i1 : i1;
            i1 = i1 >= length ? 2 * (length - 1) - i1 : i1;
            i1 = i1 < 0 ? 0 : (i1 >= length ? length - 1 : i1);
            xa[u][e] = x[i0];
            xb[u][e] = x[i1];
          }
          __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) (expcnt, lgkmcnt unconstrained)
        }
#pragma unroll
        for (int e = 0; e < E; ++e) v[u][e] = make_float2(xa[u][e] * wv[e], xb[u][e] * wv[e]);
      }
      LdsFftMulti<NFFT, E, -1, ROUNDS>::run(v, area, ltw, tid);
#pragma unroll
      for (int u = 0; u < ROUNDS; ++u) {
        // packed spectrum: entry k (0..n/2) = (Z[k], Z[n-k mod n]) as one float4
        float2* sp = reinterpret_cast<float2*>(area[u]);
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int k = tid + T * e;
          if (e < E / 2) sp[2 * k] = v[u][e];
          else sp[2 * (NFFT - k) + 1] = v[u][e];
        }
        if (tid == 0) {
          sp[1] = v[u][0];
          sp[2 * (NFFT / 2)] = v[u][E / 2];
        }
      }
#pragma unroll
      for (int u = 0; u < ROUNDS; ++u)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          xa[u][e] = ya[u][e];
          xb[u][e] = yb[u][e];
        }
      __syncthreads();  // sub-tile i's spectra ready; the store waves are done with buffer (i+1) % 2
    }
  } else {
    // ---- store waves: line task = (bin row k, 16 lanes of two frames each)
    const int sl = threadIdx.x - 64 * TWAVES;
    const int t2 = sl & 15;
    const int task = sl >> 4;
    char* pre = reinterpret_cast<char*>(out_re + (size_t)b * NB1 * n_frames);
    char* pim = reinterpret_cast<char*>(out_im + (size_t)b * NB1 * n_frames);
    float2 cre[PASSES], cim[PASSES];  // carried frames (the next sub-tile's part of this line)
    int dd[PASSES];
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int k = task + LPP * ps;
      const int o = o_tab[k < NB1 ? k : NB1 - 1];
      // forward: row k's lines start dd frames before each sub-tile; backward: dd frames after
      // it (even: n_frames and the range bounds are even, the planes 8-byte aligned)
      dd[ps] = fwd ? ((o + R0) & 31) : ((-(o + R1)) & 31);
      cre[ps] = make_float2(0.0f, 0.0f);
      cim[ps] = make_float2(0.0f, 0.0f);
    }
    typedef float f2v __attribute__((ext_vector_type(2)));
    for (int i = 0; i < steps; ++i) {
      __syncthreads();  // sub-tile i's spectra are in buffer i % 2
      const int A = fwd ? R0 + FR * i : R1 - FR * (i + 1);
      const bool first = i == 0, last = i == steps - 1;
      const float* buf = lds + (i & 1) * BUF;
#pragma unroll
      for (int ps = 0; ps < PASSES; ++ps) {
        const int k = task + LPP * ps;
        if (k >= NB1) continue;
        const int d = dd[ps];
        const int rel = fwd ? 2 * t2 - d : 2 * t2 + d;  // this lane's first frame, relative to A
        // frames of the previous sub-tile come from the carry; those lanes read the frames they
        // carry on to the next step instead
        const bool carry_lane = fwd ? rel < 0 : rel >= FR;
        const int j = carry_lane ? (fwd ? rel + FR : rel - FR) : rel;
        const float4 q = reinterpret_cast<const float4*>(buf + __umul24((unsigned)(j >> 1), (unsigned)AREA))[k];
        const float2 re = make_float2(q.x + q.z, q.y + q.w);  // frames j, j + 1: (Z[k] + conj Z[n-k]) / 2, ...
        const float2 im = make_float2(q.y - q.w, q.z - q.x);
        const float2 pr = carry_lane ? cre[ps] : re, pi = carry_lane ? cim[ps] : im;
        cre[ps] = carry_lane ? re : cre[ps];
        cim[ps] = carry_lane ? im : cim[ps];
        const int f = A + rel;
        const unsigned off = ((unsigned)k * (unsigned)n_frames + (unsigned)f) * 4u;
        if (!first && !last) {  // interior step: the line lies inside the range
          __builtin_nontemporal_store((f2v){pr.x, pr.y}, reinterpret_cast<f2v*>(pre + off));
          __builtin_nontemporal_store((f2v){pi.x, pi.y}, reinterpret_cast<f2v*>(pim + off));
          continue;
        }
        const int s = f - 2 * t2;  // this step's line: frames [s, s + 32)
        if (s >= R0 && s + 32 <= R1) {
          __builtin_nontemporal_store((f2v){pr.x, pr.y}, reinterpret_cast<f2v*>(pre + off));
          __builtin_nontemporal_store((f2v){pi.x, pi.y}, reinterpret_cast<f2v*>(pim + off));
        } else if (f >= R0 && f < R1) {  // a line shared with the neighbouring range: merged in L2
          *reinterpret_cast<float2*>(pre + off) = pr;
          *reinterpret_cast<float2*>(pim + off) = pi;
        }
        if (last && carry_lane) {
          // the range's other partial line: the frames carried on
          const int f2 = fwd ? f + 32 : f - 32;
          if (f2 >= R0 && f2 < R1) {
            const unsigned off2 = fwd ? off + 128u : off - 128u;
            *reinterpret_cast<float2*>(pre + off2) = re;
            *reinterpret_cast<float2*>(pim + off2) = im;
          }
        }
      }
    }
  }
}

// Ranges per signal for stft_binrows_kernel (even, about 256 workgroups in all, at least one
// 32-frame sub-tile per range), or 0 when its preconditions do not hold.
template <int NFFT>
static int binrows_ranges(const StftArgs& a) {
  constexpr int NB1 = NFFT / 2 + 1;
  if (a.n_bins != NB1 || a.n_frames % 2 != 0 || a.n_frames < 64 || a.length < NFFT || a.batch <= 0) return 0;
  if (a.hop < 1) return 0;
  const uintptr_t pr = reinterpret_cast<uintptr_t>(a.out_re), pi = reinterpret_cast<uintptr_t>(a.out_im);
  if ((pr & 7) != 0 || (pi & 7) != 0 || ((pr ^ pi) & 127) != 0) return 0;
  if ((long long)NB1 * a.n_frames * 4 >= (1LL << 32)) return 0;
  long long q = 2 * (long long)std::max(1.0, std::round(128.0 / (double)a.batch));
  while (q > 2 && a.n_frames / q < 32) q -= 2;
  if (a.batch * q > 0x7fffffffLL) return 0;
  return (int)q;
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
  if constexpr (NFFT == 256 || NFFT == 512) {
    // bins-major as whole lines (C2, 64 x 160000 at n_fft 512: 32.2 us against 37.6 us for the
    // fixed-tile kernel below)
    const int q = binrows_ranges<NFFT>(a);
    if (q > 0) {
      const unsigned base_mod = (unsigned)((reinterpret_cast<uintptr_t>(a.out_re) >> 2) & 31);
      hipLaunchKernelGGL((stft_binrows_kernel<NFFT>), dim3((unsigned)(a.batch * q)), dim3(BinRowsCfg<NFFT>::THREADS),
                         0, a.stream, a.signal, a.window, a.out_re, a.out_im, a.tw, a.length, a.hop, a.pad,
                         a.n_frames, q, base_mod, 0.5f * a.scale);
      return hipGetLastError();
    }
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
