// Bluestein (chirp-z) transform for arbitrary n, trnfft/fft_core.py:1285-1376.
//
// Fused path (padded length m <= 16384): one launch, one row per transform slot.  The row is
// loaded, multiplied by the chirp and zero-padded in registers, transformed forward in LDS,
// multiplied by the plan's filter spectrum H/m, transformed back, multiplied by the chirp and
// stored (first n entries only): one HBM read and one HBM write per element, against the
// reference's three separate m-point FFTs and five full-size temporaries.
//
// Split path (m > 16384, and m = 16384 when there are too few rows to fill the GPU): each row is
// spread over many workgroups with a transposed-domain four-step, m = M1 * M2, y[n1*M2 + n2],
// spectrum index k = k1 + M1*k2:
//   K1 (columns): y = x * chirp (zero past n), M1-point transform down each column n2, times
//      W_m^(n2*k1)  ->  Z[k1][n2] in the workspace;
//   K2 (rows): per row k1, M2-point forward transform (the spectrum Y[k1 + M1*k2] lands in row
//      k1), times H/m in the same permuted order, M2-point inverse transform, times W_m^-(n2*k1);
//   K3 (columns): M1-point inverse transform down each column gives p[n1*M2 + n2], times chirp
//      and the output scale, first n entries stored.
// The spectrum is never brought back to natural order: the filter multiply happens in the
// transposed domain, so the chain is three passes (the intermediate, batch*m*8 bytes, stays in
// the Infinity Cache at the BASELINE sizes) instead of two full four-step transforms.
#include "kernels.h"

namespace tfa {

// Launch shape of the fused kernel: E elements per thread, THR threads per workgroup.
template <int M, int E_, int THR>
struct BlueCfg {
  static constexpr int E = E_;
  static constexpr int T = M / E;
  static constexpr int XF = T >= THR ? 1 : THR / T;
  static constexpr int THREADS = XF * T;
  static constexpr int PADN = lds_pad(M) > 1 ? lds_pad(M) : 1;
  static constexpr bool DB = blue_db(M) && T > 64;  // double-buffered exchange (two LDS buffers per row)
  static constexpr int NBUF = DB ? 2 : 1;
};

// WRAP: the circular convolution length M is shorter than 2n - 1 by wrap = 2n - 1 - M
// (1..kBlueWrapMax).  The filter taps t and t - M (t = M - n + 1 .. n - 1) then share a slot of the
// filter (the plan sums them), which adds one extra term y[j] conj(chirp[M - k + j]) (j <= k - L,
// L = n - wrap) to the outputs k >= L and y[j] conj(chirp[k - j + M]) (j >= k + L) to the outputs
// k < wrap; both are subtracted after the inverse transform from the chirped input ends y[0, wrap),
// y[L, n) and chirp[L, n), kept in LDS.  n then exceeds M/2 by at most 8, so one more element per
// thread can hold a sample.  The corrected outputs i < wrap sit in element 0 of their threads and
// L <= i < n in elements E/2 - 1 and E/2 (L is up to 7 below M/2); the correction runs over every
// element e < E/2 + 1.
template <int M, bool REAL_IN, bool WRAP = false, int E_ = blue_epth(M), int THR = blue_threads(M)>
__global__ __launch_bounds__((BlueCfg<M, E_, THR>::THREADS)) void bluestein_fused_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re,
    float* out_im, const float2* __restrict__ chirp, const float2* __restrict__ hs,
    const float2* __restrict__ tw_f, const float2* __restrict__ tw_i, int n, long long batch,
    float scale, int wrap) {
  using C = BlueCfg<M, E_, THR>;
  constexpr int E = C::E, T = C::T;
  static_assert(!WRAP || (T > kBlueWrapMax && E >= 2),
                "wrapped lengths: the corrected outputs (i < wrap, L <= i < n) lie in elements 0, E/2 - 1 and E/2");
  __shared__ float2 lds[C::XF * C::PADN * C::NBUF];  // interleaved (re, im) exchange
  __shared__ float2 ends_all[WRAP ? C::XF * 3 * kBlueWrapMax : 1];  // per row: y[0, wrap), y[L, n), chirp[L, n)
  // short rows (M <= 64, up to 8 threads per row): a thread's own loads would touch a different
  // cache line per lane (rows of n <= 32 samples), so the workgroup's XF rows move between HBM and
  // LDS as one contiguous run of rows * n floats per plane (row r at r * n), NS coalesced steps
  constexpr bool STG = T <= 8 && !WRAP;
  constexpr int NS = (C::XF * (M / 2) + C::THREADS - 1) / C::THREADS;
  __shared__ float2 stg[STG ? C::XF * (M / 2) : 1];
  const long long r0 = (long long)blockIdx.x * C::XF;
  const int srows = STG ? (int)(batch - r0 < C::XF ? batch - r0 : C::XF) : 0;
  const int scnt = srows * n;
  const size_t g0 = (size_t)r0 * n;
  const int tid = threadIdx.x % T;
  const int xf = threadIdx.x / T;
  const long long b = (long long)blockIdx.x * C::XF + xf;
  const bool valid = b < batch;
  const size_t base = (size_t)b * n;
  // a slot past the last row reads the last row (its results are not stored)
  const size_t lbase = (size_t)(valid ? b : batch - 1) * n;
  const int L = n - wrap;
  float2* ends = ends_all + (WRAP ? xf * 3 * kBlueWrapMax : 0);

  // every workgroup of the launch runs the same phase at the same time, so nothing hides a
  // table load issued where it is used: with up to 8 elements per thread the chirp is loaded
  // once (it multiplies both the input and the output) and the filter spectrum is requested
  // before the forward transform; with 12 (the mixed-radix lengths) the filter spectrum is
  // requested before the forward transform and the output chirp before the inverse one; with 16
  // the extra registers would spill, and both tables are read where they are used.
  // n <= M/2 (M >= 2n - 1), so element e of a thread can hold a sample only for e < E/2: the
  // upper half of the forward input is zero at compile time and the upper half of the inverse
  // output is never needed (its last-pass arithmetic is dead code).
  constexpr int EH = (E / 2 > 0 ? E / 2 : 1) + (WRAP ? 1 : 0);
  constexpr bool PRE = E <= 8;
  constexpr bool PRE2 = E == 12;
  float2 v[E], ch[PRE ? EH : 1], hv[PRE || PRE2 ? E : 1];
  // the row's loads at a clamped index and without branches, so that every element's load issues
  // before the first wait (under `if (i < n)` the compiler waited for each load before issuing
  // the next one); non-temporal: every row is read and written once (C3b 18.4 -> 17.3 us, C3a
  // 12.0 -> 11.4)
  float2 cl[EH], xl[EH];
  if constexpr (STG) {
    float sr[NS], si[NS];
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int i = (int)threadIdx.x + C::THREADS * u;
      const int ic = i < scnt ? i : scnt - 1;
      sr[u] = ld_stream(in_re + g0 + ic);
      si[u] = REAL_IN ? 0.0f : ld_stream(in_im + g0 + ic);
    }
    __builtin_amdgcn_sched_barrier(0);  // (else the scheduler pairs each load with its write)
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int i = (int)threadIdx.x + C::THREADS * u;
      if (i < scnt) stg[i] = make_float2(sr[u], si[u]);
    }
    __syncthreads();
    // (rows past the batch read the staging area's stale entries: transformed, never stored)
#pragma unroll
    for (int e = 0; e < EH; ++e) {
      const int i = tid + T * e;
      const int ic = i < n ? i : n - 1;
      cl[e] = chirp[ic];
      xl[e] = stg[xf * n + ic];
    }
  } else {
#pragma unroll
    for (int e = 0; e < EH; ++e) {
      const int i = tid + T * e;
      const int ic = i < n ? i : n - 1;
      cl[e] = chirp[ic];
      xl[e] = make_float2(ld_stream(in_re + lbase + ic), REAL_IN ? 0.0f : ld_stream(in_im + lbase + ic));
    }
  }
  if constexpr (PRE || PRE2) {
#pragma unroll
    for (int e = 0; e < E; ++e) hv[PRE || PRE2 ? e : 0] = hs[tid + T * e];
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid + T * e;
    float2 y = make_float2(0.0f, 0.0f);
    if (e < EH) {
      // (a padded slot multiplies the clamped sample by a zero chirp: zero for finite input)
      const float2 c = i < n ? cl[e < EH ? e : 0] : make_float2(0.0f, 0.0f);
      if constexpr (PRE) ch[PRE ? e : 0] = c;
      y = cmul(xl[e < EH ? e : 0], c);
      if constexpr (WRAP) {
        // (read after the transforms, whose exchanges synchronise the workgroup)
        if (i < wrap) ends[i] = y;
        if (i >= L && i < n) {
          ends[kBlueWrapMax + i - L] = y;
          ends[2 * kBlueWrapMax + i - L] = c;
        }
      }
    }
    v[e] = y;
  }
  float* my = reinterpret_cast<float*>(lds + xf * C::PADN * C::NBUF);
  constexpr bool PF = blue_pf(M);
  LdsFft<M, E, -1, (T <= 64), false, true, PF, C::DB>::run(v, my, nullptr, tw_f, tid);
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = cmul(v[e], PRE || PRE2 ? hv[PRE || PRE2 ? e : 0] : hs[tid + T * e]);
  float2 ch2[PRE2 ? EH : 1];
  if constexpr (PRE2) {
#pragma unroll
    for (int e = 0; e < EH; ++e) {
      const int i = tid + T * e;
      ch2[e] = i < n ? chirp[i] : make_float2(0.0f, 0.0f);
    }
  }
  LdsFft<M, E, 1, (T <= 64), false, true, PF, C::DB>::run(v, my, nullptr, tw_i, tid);
  if constexpr (STG) {
    __syncthreads();  // every row's staged input is read
#pragma unroll
    for (int e = 0; e < EH; ++e) {
      const int i = tid + T * e;
      if (i < n) {
        const float2 y = cmul(v[e], PRE ? ch[PRE ? e : 0] : chirp[i]);
        stg[xf * n + i] = make_float2(y.x * scale, y.y * scale);
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int i = (int)threadIdx.x + C::THREADS * u;
      if (i < scnt) {
        const float2 y = stg[i];
        st_stream(out_re + g0 + i, y.x);
        st_stream(out_im + g0 + i, y.y);
      }
    }
    return;
  }
  if (valid) {
#pragma unroll
    for (int e = 0; e < EH; ++e) {
      const int i = tid + T * e;
      if (i < n) {
        float2 cv = v[e];
        if constexpr (WRAP) {
          const float2* yl = ends;
          const float2* yh = ends + kBlueWrapMax;
          const float2* ct = ends + 2 * kBlueWrapMax;
          if (i < wrap) {  // extra terms y[L + c] conj(chirp[L + wrap - 1 + i - c]), c = i .. wrap-1
            for (int c = i; c < wrap; ++c) {
              const float2 t = ct[wrap - 1 + i - c];
              cv = csub(cv, cmul(yh[c], make_float2(t.x, -t.y)));
            }
          }
          if (i >= L) {  // extra terms y[j] conj(chirp[L + wrap - 1 - a + j]), j = 0 .. a, a = i - L
            const int a = i - L;
            for (int j = 0; j <= a; ++j) {
              const float2 t = ct[wrap - 1 - a + j];
              cv = csub(cv, cmul(yl[j], make_float2(t.x, -t.y)));
            }
          }
        }
        const float2 y = cmul(cv, PRE ? ch[PRE ? e : 0] : PRE2 ? ch2[PRE2 ? e : 0] : chirp[i]);
        st_stream(out_re + base + i, y.x * scale);
        st_stream(out_im + base + i, y.y * scale);
      }
    }
  }
}

// Two-level fused Bluestein at M = 2048, 4096, 8192 and 16384: each row is R = M / B wavefronts of
// B points (B = 512 with 8 elements per lane; at 16384 B = 1024 with 16 per lane, 16 waves, and
// the filter spectrum and output chirp read where used so that the transforms keep their
// registers: 80 -> 57.5 us for 680 rows of n = 6145, 56 -> 42 for 300 wrapped rows of 8193,
// against the one-level kernel).  The one-level kernel above synchronises the whole workgroup at every radix pass
// (about ten barriers per row at M = 8192, and the waves of a one-row-per-CU launch spend most
// of their cycles waiting), so here the length splits as M = R x 512, n = 512 n_a + n_b,
// k = k_a + R k_b:
//   forward: thread t of the row holds x[t + T e] (T = M / 8) and transforms over the n_a it holds
//     in registers (R = 4: two 4-point DFTs, columns n_b = t and t + 256; R = 8: the whole column
//     n_b = t; R = 16: the samples n_a = 2e + p of column n_b = t % 512, p = t / 512, the 8-point
//     half of the 16-point DFT); one exchange through LDS gives wave w = k_a its values for all
//     512 n_b (for R = 16 the radix-2 half: Y_0[k'] + (-1)^q W_16^k' Y_1[k'], w = k' + 8q), times
//     W_M^(n_b k_a); a 512-point transform inside the wave (wave-local exchanges only) leaves
//     X[k_a + R k_b] with k_b = lane + 64 e;
//   the filter spectrum is applied in that order (the plan stores H/M permuted to it), then the
//     wave's 512-point inverse transform, times W_M^(-n_b k_a), written into the wave's own
//     exchange area;
//   inverse: one exchange back gives each thread the R values Z[k_a][n_b] of its columns; the
//     inverse DFT over k_a in registers (for R = 16: the pairs (Z[k'] +- Z[k' + 8]) times
//     W_16^(-p k') and an 8-point inverse DFT) gives y[t + T e]: natural order again for the
//     chirp, the wrap correction and the stores.
// Two workgroup barriers per row (one row per workgroup).  tw_f / tw_i: the 512-point transform's
// table (tfa::make_shape(512, 8)), then from entry kBlue2lTwOff the rows W_M^(+-n_b w), w < R,
// n_b < 512.  A launch of C3a's 1024 rows at M = 2048 is one workgroup per SIMD, so the row's
// waits make up the kernel's time, and the loads in flight at the first exchange set the first
// wait: the cross factor W_M^(w (l + 64 e)) is formed as W_M^(w l) (one vector load) times the
// wave-uniform W_M^(64 w e) (scalar loads) rather than loaded per element.  Measured (in-run):
// 256 x 4099 (M = 8192, wrapped) 13.7 -> 12.3 us against the one-level kernel, 11.7 with the
// formed cross factor; 1024 x 1000 (M = 2048) 10.6 (one-level kernel, or two-level with loaded
// cross factors) -> 9.8; 512 x 1025 9.3 -> 8.2.  Slower where the launch is one round of
// workgroups: the 512-point transform's twiddles loaded into registers with the row (1024 x 1000
// 10.2 us, 256 x 4099 13.3-13.7, either table layout) or staged in LDS (11.3 / 12.6: the staging
// stores wait for every load issued before them); both win only for many rows per CU
// (4096 x 800: 28.3-29.4 against 31.9 us).
template <int M>
struct Blue2lCfg {
  static constexpr int B = blue_2l_b(M), E = blue_2l_e(M), R = M / B, T = M / E, PB = lds_pad(B);
  static constexpr int TWOFF = blue_2l_twoff(M);
  static_assert(make_shape(B, E).twoff[make_shape(B, E).npass] + 2 <= TWOFF, "the wave table fits before the cross rows");
};
template <int M, bool REAL_IN, bool WRAP>
__global__ __launch_bounds__(Blue2lCfg<M>::T) void bluestein_2l_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re, float* out_im,
    const float2* __restrict__ chirp, const float2* __restrict__ hs, const float2* __restrict__ tw_f,
    const float2* __restrict__ tw_i, int n, long long batch, float scale, int wrap) {
  using C = Blue2lCfg<M>;
  constexpr int R = C::R, E = C::E, T = C::T, B = C::B, PB = C::PB;
  constexpr int TWOFF = C::TWOFF;
  // the register DFT over n_a: half of it per thread (R = 2E, two threads per column), all of it
  // (R = E) or two quarter-length ones (R = E / 2, a thread holds two columns)
  static_assert((R == 2 * E && E == 8) || R == E || (R * 2 == E && E == 8), "two-level Bluestein lengths");
  constexpr bool PS = R == 2 * E;  // two threads per column (the radix-2 split of the R-point DFT)
  // with R <= E wave w reads back only region w of the forward exchange, so the regions are the
  // waves' own transform areas (stride PB); R = 2E reads two regions per wave (its own buffer)
  constexpr bool ALIAS = R <= E;
  constexpr int XS = ALIAS ? PB : B;
  __shared__ float2 xbuf[ALIAS ? 2 : M];  // the forward exchange (R = 2E)
  __shared__ float2 warea[R * PB];  // each wave's B-point exchange area; the inverse exchange
  float2* const xb = ALIAS ? warea : xbuf;
  __shared__ float2 ends[WRAP ? 3 * kBlueWrapMax : 1];  // y[0, wrap), y[L, n), chirp[L, n)
  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63;
  const size_t base = (size_t)blockIdx.x * n;
  const int L = n - wrap;
  // n <= M/2 (+ up to 8 wrapped): element e of a thread can hold a sample only for e < EH
  constexpr int EH = E / 2 + (WRAP ? 1 : 0);
  // the cross factor W_M^(w (l + 64 e)) = W_M^(w l) W_M^(64 w e): one vector load and the
  // wave-uniform second factors (scalar loads, issued first so they land during the row's loads)
  const int wu = __builtin_amdgcn_readfirstlane(w);
  float2 cf[E];
#pragma unroll
  for (int e = 1; e < E; ++e) cf[e] = tw_f[TWOFF + wu * B + 64 * e];
  // the row's loads at a clamped index, without branches: every element's loads are in flight
  // before the first wait (a load under `if (i < n)` is waited for before the next one issues)
  float2 ch[EH], xin[EH];
#pragma unroll
  for (int e = 0; e < EH; ++e) {
    const int i = tid + T * e;
    const int ic = i < n ? i : n - 1;
    // at 8192 and 16384 points (unwrapped) a wave none of whose lanes holds a sample in element e
    // skips its loads with a wave-uniform branch (n <= 3072 leaves element 3 empty at 8192 points,
    // n <= 7168 element 7 at 16384: 2100 x 1997 64.3 -> 62.2 us, 6145 x 680 57.5 -> 56.3); the
    // wrapped kernels (C3b: only the first wave has samples past M/2) measured 1 % slower with the
    // branches, and at 2048 / 4096 points they kept the scheduler from issuing the filter
    // spectrum's loads before the row's waits
    if ((M != 8192 && M != 16384) || WRAP || e == 0 || T * e + wu * 64 < n) {
      ch[e] = chirp[ic];
      xin[e] = make_float2(ld_stream(in_re + base + ic), REAL_IN ? 0.0f : ld_stream(in_im + base + ic));
    } else {
      ch[e] = make_float2(0.0f, 0.0f);
      xin[e] = make_float2(0.0f, 0.0f);
    }
  }
  const float2 tb = tw_f[TWOFF + w * B + l];
  // E = 16: the filter spectrum and the output chirp are read where used and the cross factors
  // formed where used (held through the transforms, they spilled registers)
  constexpr bool HOLD = E <= 8;
  float2 hv[HOLD ? E : 1];
  // at 8192 points (16 waves, one workgroup per CU) the filter spectrum is requested after the
  // first exchange: requested with the row, its 64 KB per workgroup doubled the cache traffic of
  // the load phase that every wave waits for (256 x 4099 11.17 -> 11.02 us, 3000 x 1398 51.7 ->
  // 50.6); at 2048 / 4096 points (several workgroups per CU, whose phases overlap) that measured
  // 1-2 % slower
  constexpr bool HV_LATE = HOLD && M == 8192;
  if constexpr (HOLD && !HV_LATE) {
#pragma unroll
    for (int e = 0; e < E; ++e) hv[HOLD ? e : 0] = hs[tid + T * e];
  }
  // the uniform factors are waited for here, while the vector loads are in flight (left to the
  // compiler, the wrapped kernels issued them just before the first barrier, which then waited)
#pragma unroll
  for (int e = 1; e < E; ++e) asm volatile("" ::"s"(cf[e].x), "s"(cf[e].y));
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid + T * e;
    float2 y = make_float2(0.0f, 0.0f);
    if (e < EH) {
      // (a padded slot multiplies the clamped sample by a zero chirp: zero for finite input)
      const float2 c = i < n ? ch[e < EH ? e : 0] : make_float2(0.0f, 0.0f);
      ch[e < EH ? e : 0] = c;
      y = cmul(xin[e < EH ? e : 0], c);
      if constexpr (WRAP) {
        if (i < wrap) ends[i] = y;
        if (i >= L && i < n) {
          ends[kBlueWrapMax + i - L] = y;
          ends[2 * kBlueWrapMax + i - L] = c;
        }
      }
    }
    v[e] = y;
  }
  float2 tcr[HOLD ? E : 1];
  auto cross = [&](int e) { return e == 0 ? tb : cmul(tb, cf[e]); };
  if constexpr (HOLD) {
#pragma unroll
    for (int e = 0; e < E; ++e) tcr[HOLD ? e : 0] = cross(e);
  }
  // W_16^j = (cos, -sin)(2 pi j / 16) for the forward sign
  constexpr float kC16[8] = {(float)cos2pi(0, 16), (float)cos2pi(1, 16), (float)cos2pi(2, 16), (float)cos2pi(3, 16),
                             (float)cos2pi(4, 16), (float)cos2pi(5, 16), (float)cos2pi(6, 16), (float)cos2pi(7, 16)};
  constexpr float kS16[8] = {(float)sin2pi(0, 16), (float)sin2pi(1, 16), (float)sin2pi(2, 16), (float)sin2pi(3, 16),
                             (float)sin2pi(4, 16), (float)sin2pi(5, 16), (float)sin2pi(6, 16), (float)sin2pi(7, 16)};
  // forward, in registers over the n_a each thread holds, then the exchange: xb[k_a * XS + n_b]
  // (R = 2E: xb[(p * E + k') * XS + n_b] holds the half transform Y_p[k'], times W_16^k' for p = 1)
  if constexpr (PS) {
    Dft<E, -1>::run(v);
    // p = 1 (the upper B-thread half, wave-uniform) applies the combination's twiddle W_16^k'
    // with compile-time constants here, so the reading waves only add or subtract the halves
    if (wu >= B / 64) {
      v[1] = twiddle_const<1, 16, -1>(v[1]);
      v[2] = twiddle_const<2, 16, -1>(v[2]);
      v[3] = twiddle_const<3, 16, -1>(v[3]);
      v[4] = twiddle_const<4, 16, -1>(v[4]);
      v[5] = twiddle_const<5, 16, -1>(v[5]);
      v[6] = twiddle_const<6, 16, -1>(v[6]);
      v[7] = twiddle_const<7, 16, -1>(v[7]);
    }
    const int p = tid / B, nb = tid % B;
#pragma unroll
    for (int k = 0; k < E; ++k) xb[(p * E + k) * XS + nb] = v[k];
  } else if constexpr (R == E) {
    Dft<E, -1>::run(v);
#pragma unroll
    for (int k = 0; k < E; ++k) xb[k * XS + tid] = v[k];
  } else {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float2 u[4] = {v[c], v[c + 2], v[c + 4], v[c + 6]};
      Dft<4, -1>::run(u);
#pragma unroll
      for (int k = 0; k < 4; ++k) xb[k * XS + tid + T * c] = u[k];
    }
  }
  __syncthreads();
  if constexpr (HV_LATE) {
#pragma unroll
    for (int e = 0; e < E; ++e) hv[HOLD ? e : 0] = hs[tid + T * e];
  }
  if constexpr (PS) {
    // Y[kq + 8 j] = Y_0[kq] + (-1)^j W_16^kq Y_1[kq] (the twiddle already applied by the writers)
    const int kq = wu & 7;
    const float sg = wu >= 8 ? -1.0f : 1.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float2 y0 = xb[kq * XS + l + 64 * e];
      const float2 y1 = xb[(8 + kq) * XS + l + 64 * e];
      v[e] = cmul(make_float2(fmaf(sg, y1.x, y0.x), fmaf(sg, y1.y, y0.y)), tcr[HOLD ? e : 0]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = cmul(xb[w * XS + l + 64 * e], HOLD ? tcr[HOLD ? e : 0] : cross(e));
  }
  // (aliased: the wave's transform overwrites region w, which only this wave has read since the
  // barrier)
  float* wa = reinterpret_cast<float*>(warea + w * PB);
  constexpr bool PF = E <= 8;  // the next pass's twiddles prefetched (E = 16: registers)
  LdsFft<B, E, -1, true, false, true, PF>::run(v, wa, nullptr, tw_f, l);
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = cmul(v[e], HOLD ? hv[HOLD ? e : 0] : hs[tid + T * e]);
  LdsFft<B, E, 1, true, false, true, PF>::run(v, wa, nullptr, tw_i, l);
  // the wave's own exchange area takes its result (its last reads of the area came before the
  // transform's final wave barrier), so no barrier guards the first exchange's buffer
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float2 t = HOLD ? tcr[HOLD ? e : 0] : cross(e);
    warea[w * PB + l + 64 * e] = cmul(v[e], make_float2(t.x, -t.y));
  }
  __syncthreads();
  // inverse over k_a in registers: y[t + T e] into v[e]
  if constexpr (PS) {
    // u[k'] = Z[k'] + Z[k' + 8] (p = 0) or (Z[k'] - Z[k' + 8]) W_16^-k' (p = 1), then the 8-point
    // inverse DFT over k' gives y[B (2e + p) + n_b]
    const int p = tid / B, nb = tid % B;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float2 z0 = warea[k * PB + nb], z1 = warea[(k + 8) * PB + nb];
      if (p == 0) v[k] = cadd(z0, z1);
      else v[k] = cmul(csub(z0, z1), make_float2(kC16[k], kS16[k]));  // W_16^-k (inverse sign)
    }
    Dft<8, 1>::run(v);
  } else if constexpr (R == E) {
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = warea[k * PB + tid];
    Dft<E, 1>::run(v);
  } else {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float2 u[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) u[k] = warea[k * PB + tid + T * c];
      Dft<4, 1>::run(u);
#pragma unroll
      for (int a = 0; a < 4; ++a) v[2 * a + c] = u[a];
    }
  }
#pragma unroll
  for (int e = 0; e < EH; ++e) {
    const int i = tid + T * e;
    if (i < n) {
      float2 cv = v[e];
      if constexpr (WRAP) {
        const float2* yl = ends;
        const float2* yh = ends + kBlueWrapMax;
        const float2* ct = ends + 2 * kBlueWrapMax;
        if (i < wrap) {
          for (int c = i; c < wrap; ++c) {
            const float2 t = ct[wrap - 1 + i - c];
            cv = csub(cv, cmul(yh[c], make_float2(t.x, -t.y)));
          }
        }
        if (i >= L) {
          const int a = i - L;
          for (int j = 0; j <= a; ++j) {
            const float2 t = ct[wrap - 1 - a + j];
            cv = csub(cv, cmul(yl[j], make_float2(t.x, -t.y)));
          }
        }
      }
      const float2 y = cmul(cv, HOLD ? ch[e] : chirp[i]);  // (E = 16: read again, not held)
      st_stream(out_re + base + i, y.x * scale);
      st_stream(out_im + base + i, y.y * scale);
    }
  }
}

template <int M, bool WRAP>
static hipError_t launch_blue_mw(const BluesteinArgs& a) {
  if constexpr (blue_2l(M)) {
    using C2 = Blue2lCfg<M>;
    const long long blocks = a.batch;  // one row per workgroup
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    if (a.in_im == nullptr)
      hipLaunchKernelGGL((bluestein_2l_kernel<M, true, WRAP>), dim3((unsigned)blocks), dim3(C2::T), 0, a.stream,
                         a.in_re, a.in_im, a.out_re, a.out_im, a.chirp, a.hs, a.tw_f, a.tw_i, a.n, a.batch, a.scale,
                         a.wrap);
    else
      hipLaunchKernelGGL((bluestein_2l_kernel<M, false, WRAP>), dim3((unsigned)blocks), dim3(C2::T), 0, a.stream,
                         a.in_re, a.in_im, a.out_re, a.out_im, a.chirp, a.hs, a.tw_f, a.tw_i, a.n, a.batch, a.scale,
                         a.wrap);
    return hipGetLastError();
  } else {
    using C = BlueCfg<M, blue_epth(M), blue_threads(M)>;
    const long long blocks = (a.batch + C::XF - 1) / C::XF;
    if (a.in_im == nullptr)
      hipLaunchKernelGGL((bluestein_fused_kernel<M, true, WRAP>), dim3((unsigned)blocks), dim3(C::THREADS), 0,
                         a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.chirp, a.hs, a.tw_f, a.tw_i,
                         a.n, a.batch, a.scale, a.wrap);
    else
      hipLaunchKernelGGL((bluestein_fused_kernel<M, false, WRAP>), dim3((unsigned)blocks), dim3(C::THREADS),
                         0, a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.chirp, a.hs, a.tw_f,
                         a.tw_i, a.n, a.batch, a.scale, a.wrap);
    return hipGetLastError();
  }
}

template <int M>
static hipError_t launch_blue_m(const BluesteinArgs& a) {
  if (a.wrap == 0) return launch_blue_mw<M, false>(a);
  if constexpr (blue_wrap_ok(M)) {
    // wrapped lengths: n = (M + 1 + wrap) / 2 holds one element per thread beyond M/2
    if (a.wrap < 0 || a.wrap > kBlueWrapMax || 2 * a.n - 1 - a.wrap != M) return hipErrorInvalidValue;
    return launch_blue_mw<M, true>(a);
  } else {
    return hipErrorInvalidValue;
  }
}

// Bluestein down a strided axis: x viewed as (outer, n, S); every column of n elements at stride
// S runs the fused kernel's steps (chirp, zero padding to M, FFT_M, times H/M, IFFT_M, chirp,
// scale) in LDS, C adjacent columns per workgroup so each access instruction covers C consecutive
// floats.  Replaces the transpose round trip of trnfft/api.py:496-516 for non-power-of-two axes.
template <int M, bool REAL_IN, int C = fourstep_tile(M)>
__global__ __launch_bounds__(C * (M / lds_epth(M))) void strided_blue_kernel(
    const float* in_re, const float* in_im, float* out_re, float* out_im, const float2* __restrict__ chirp,
    const float2* __restrict__ hs, const float2* __restrict__ tw_f, const float2* __restrict__ tw_i, long long stride,
    int tiles_per_block, int n, float scale) {
  // in place is allowed: a workgroup reads all of its columns before its first barrier and no
  // other workgroup touches them
  constexpr int E = lds_epth(M), T = M / E;
  constexpr int PADN = lds_pad(M) + 1;
  __shared__ float2 lds[C * PADN];  // interleaved (re, im) exchange, one column per region
  const int c = threadIdx.x % C;  // column within the tile (fast across lanes)
  const int t = threadIdx.x / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_block;
  const long long col = (tile % tiles_per_block) * C + c;
  const bool valid = col < stride;
  const size_t base = (size_t)b * n * stride + col;
  // loads at a clamped column and index, without branches, so that every element's loads issue
  // before the first wait; the padded slots and the columns past the last take a zero chirp
  const size_t lbase = (size_t)b * n * stride + (valid ? col : stride - 1);
  float2 xl[E], cl[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = t + T * e;
    const int ic = i < n ? i : n - 1;
    const size_t s = lbase + (size_t)ic * stride;
    xl[e] = make_float2(in_re[s], REAL_IN ? 0.0f : in_im[s]);
    cl[e] = chirp[ic];
  }
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = t + T * e;
    v[e] = cmul(xl[e], valid && i < n ? cl[e] : make_float2(0.0f, 0.0f));
  }
  float* my = reinterpret_cast<float*>(lds + c * PADN);
  // next-pass twiddle prefetch from M = 256 (1000-point columns 49.7 -> 46.2 us, the 480 axis of
  // 64 x 480 x 640 189.8 -> 184.3; 1.6 % slower at M = 32)
  constexpr bool PF = M >= 256;
  LdsFft<M, E, -1, false, false, true, PF>::run(v, my, nullptr, tw_f, t);
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = cmul(v[e], hs[t + T * e]);
  LdsFft<M, E, 1, false, false, true, PF>::run(v, my, nullptr, tw_i, t);
  if (!valid) return;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = t + T * e;
    if (i < n) {
      const float2 y = cmul(v[e], chirp[i]);
      const size_t o = base + (size_t)i * stride;
      out_re[o] = y.x * scale;  // plain stores: row segments of C floats (L2 merges partial lines)
      out_im[o] = y.y * scale;
    }
  }
}

template <int M>
static hipError_t launch_strided_blue_m(const StridedBlueArgs& a) {
  constexpr int C = fourstep_tile(M), T = M / lds_epth(M);
  const long long tiles = (a.stride + C - 1) / C;
  const long long blocks = a.outer * tiles;
  if (a.in_im == nullptr)
    hipLaunchKernelGGL((strided_blue_kernel<M, true>), dim3((unsigned)blocks), dim3(C * T), 0, a.stream, a.in_re,
                       a.in_im, a.out_re, a.out_im, a.chirp, a.hs, a.tw_f, a.tw_i, a.stride, (int)tiles, a.n, a.scale);
  else
    hipLaunchKernelGGL((strided_blue_kernel<M, false>), dim3((unsigned)blocks), dim3(C * T), 0, a.stream, a.in_re,
                       a.in_im, a.out_re, a.out_im, a.chirp, a.hs, a.tw_f, a.tw_i, a.stride, (int)tiles, a.n, a.scale);
  return hipGetLastError();
}

hipError_t launch_strided_bluestein(int m, const StridedBlueArgs& a) {
  switch (m) {
    case 4: return launch_strided_blue_m<4>(a);
    case 8: return launch_strided_blue_m<8>(a);
    case 16: return launch_strided_blue_m<16>(a);
    case 32: return launch_strided_blue_m<32>(a);
    case 64: return launch_strided_blue_m<64>(a);
    case 128: return launch_strided_blue_m<128>(a);
    case 256: return launch_strided_blue_m<256>(a);
    case 512: return launch_strided_blue_m<512>(a);
    case 1024: return launch_strided_blue_m<1024>(a);
    case 2048: return launch_strided_blue_m<2048>(a);
    case 4096: return launch_strided_blue_m<4096>(a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bluestein_fused(int m, const BluesteinArgs& a) {
  switch (m) {
    case 4: return launch_blue_m<4>(a);
    case 8: return launch_blue_m<8>(a);
    case 16: return launch_blue_m<16>(a);
    case 32: return launch_blue_m<32>(a);
    case 64: return launch_blue_m<64>(a);
    case 128: return launch_blue_m<128>(a);
    case 256: return launch_blue_m<256>(a);
    case 512: return launch_blue_m<512>(a);
    case 1024: return launch_blue_m<1024>(a);
    case 2048: return launch_blue_m<2048>(a);
    case 4096: return launch_blue_m<4096>(a);
    case 8192: return launch_blue_m<8192>(a);
    case 16384: return launch_blue_m<16384>(a);
    case 768: return launch_blue_m<768>(a);
    case 1536: return launch_blue_m<1536>(a);
    case 3072: return launch_blue_m<3072>(a);
    case 9216: return launch_blue_m<9216>(a);
    case 12288: return launch_blue_m<12288>(a);
    default: return hipErrorInvalidValue;
  }
}

// ---- split path ---------------------------------------------------------------------------------

// W_m^j from the two-level table (j < m); conjugated when CONJ.
template <bool CONJ>
__device__ __forceinline__ float2 root_m(const float2* __restrict__ lo, const float2* __restrict__ hi, unsigned j,
                                         int lo_bits) {
  const float2 w = cmul(lo[j & ((1u << lo_bits) - 1)], hi[j >> lo_bits]);
  return CONJ ? make_float2(w.x, -w.y) : w;
}

// v[e] *= W_m^(f * (t + T*e)) (conjugated when CONJ), e < E.  The roots are read as
// W^(f (t + T*TF*a)) * W^(f T j) for e = TF*a + j: E/TF + TF - 1 two-level table reads per thread
// instead of E (the table reads are scattered gathers; the four-step column pass measured 15 -> 3
// us with this factoring).  Index products wrap modulo 2^32, a multiple of m.
template <int E, int T, bool CONJ>
__device__ __forceinline__ void mul_roots(float2 (&v)[E], const float2* __restrict__ lo,
                                          const float2* __restrict__ hi, unsigned f, unsigned t, unsigned mask,
                                          int lo_bits) {
  constexpr int TF = E < 4 ? E : 4;
  float2 q[TF];
#pragma unroll
  for (int j = 1; j < TF; ++j) q[j] = root_m<CONJ>(lo, hi, (f * (unsigned)(T * j)) & mask, lo_bits);
#pragma unroll
  for (int a = 0; a < E / TF; ++a) {
    const float2 p = root_m<CONJ>(lo, hi, (f * (t + (unsigned)(T * TF * a))) & mask, lo_bits);
    v[TF * a] = cmul(v[TF * a], p);
#pragma unroll
    for (int j = 1; j < TF; ++j) v[TF * a + j] = cmul(v[TF * a + j], cmul(p, q[j]));
    __builtin_amdgcn_sched_barrier(0);  // one group of table reads in flight at a time (registers)
  }
}

// Column passes: C adjacent columns of one row's M1 x M2 view per workgroup (coalesced across
// columns), LDS Stockham down the column.
template <int M1>
struct BlueColCfg {
  static constexpr int E = blue_col_epth(M1);
  static constexpr int T = M1 / E;
  // the strided-pass tile, narrowed when fewer elements per thread need more threads per column
  static constexpr int C = fourstep_tile(M1) * T > 1024 ? 1024 / T : fourstep_tile(M1);
  static constexpr int PADN = lds_pad(M1) + 1;
};

template <int M1, bool REAL_IN>
__global__ __launch_bounds__((BlueColCfg<M1>::C * BlueColCfg<M1>::T)) void blue_col_fwd_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* __restrict__ ws_re,
    float* __restrict__ ws_im, const float2* __restrict__ chirp, const float2* __restrict__ tw,
    const float2* __restrict__ lo, const float2* __restrict__ hi, int lo_bits, int n, int m2, int tiles) {
  using G = BlueColCfg<M1>;
  constexpr int E = G::E, T = G::T, C = G::C, PADN = G::PADN;
  __shared__ float2 lds[C * PADN];  // interleaved (re, im) exchange
  const int c = threadIdx.x % C, t = threadIdx.x / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles;
  const int col = (int)(tile % tiles) * C + c;
  const unsigned m = (unsigned)M1 * (unsigned)m2;
  // loads at a clamped index without branches (every element's loads issue before the first
  // wait); the slots past n take a zero chirp
  float2 xl[E], cl[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = (t + T * e) * m2 + col;
    const int ic = i < n ? i : n - 1;
    const size_t s = (size_t)b * n + ic;
    xl[e] = make_float2(in_re[s], REAL_IN ? 0.0f : in_im[s]);
    cl[e] = chirp[ic];
  }
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e)
    v[e] = cmul(xl[e], (t + T * e) * m2 + col < n ? cl[e] : make_float2(0.0f, 0.0f));
  LdsFft<M1, E, -1, false, false, true, blue_split_pf(M1)>::run(v, reinterpret_cast<float*>(lds + c * PADN), nullptr, tw, t);
  mul_roots<E, T, false>(v, lo, hi, (unsigned)col, (unsigned)t, m - 1, lo_bits);  // W_m^(col*k1)
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k1 = t + T * e;
    const size_t o = (size_t)b * m + (size_t)k1 * m2 + col;
    st_stream(ws_re + o, v[e].x);
    st_stream(ws_im + o, v[e].y);
  }
}

template <int M1>
__global__ __launch_bounds__((BlueColCfg<M1>::C * BlueColCfg<M1>::T)) void blue_col_inv_kernel(
    const float* __restrict__ ws_re, const float* __restrict__ ws_im, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ chirp, const float2* __restrict__ tw, int n, int m2,
    int tiles, float scale) {
  using G = BlueColCfg<M1>;
  constexpr int E = G::E, T = G::T, C = G::C, PADN = G::PADN;
  __shared__ float2 lds[C * PADN];  // interleaved (re, im) exchange
  const int c = threadIdx.x % C, t = threadIdx.x / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles;
  const int col = (int)(tile % tiles) * C + c;
  const size_t m = (size_t)M1 * m2;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t s = (size_t)b * m + (size_t)(t + T * e) * m2 + col;
    v[e] = make_float2(ld_stream(ws_re + s), ld_stream(ws_im + s));
  }
  LdsFft<M1, E, 1, false, false, true, blue_split_pf(M1)>::run(v, reinterpret_cast<float*>(lds + c * PADN), nullptr, tw, t);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = (t + T * e) * m2 + col;
    if (i < n) {
      const float2 y = cmul(v[e], chirp[i]);
      const size_t o = (size_t)b * n + i;
      out_re[o] = y.x * scale;
      out_im[o] = y.y * scale;
    }
  }
}

// Row pass: forward M2-point transform, filter, inverse M2-point transform, inverse twiddle, in
// place in the workspace (rows of M2 contiguous elements; batched-c2c launch shape).
template <int M2>
__global__ __launch_bounds__(C2cThreads<M2>::THREADS) void blue_row_kernel(
    float* __restrict__ ws_re, float* __restrict__ ws_im, const float2* __restrict__ hp,
    const float2* __restrict__ tw_f, const float2* __restrict__ tw_i, const float2* __restrict__ lo,
    const float2* __restrict__ hi, int lo_bits, int m1) {
  using C = C2cThreads<M2>;
  constexpr int E = C::E, T = C::T;
  constexpr bool WL = T <= 64;
  __shared__ float2 lds[C::XF * C::PADN];  // interleaved (re, im) exchange
  const int tid = threadIdx.x % T, xf = threadIdx.x / T;
  const long long row = (long long)blockIdx.x * C::XF + xf;  // (batch, k1)
  const int k1 = (int)(row % m1);
  const unsigned m = (unsigned)m1 * (unsigned)M2;
  float* pr = ws_re + (size_t)row * M2 + tid;
  float* pi = ws_im + (size_t)row * M2 + tid;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = make_float2(pr[T * e], pi[T * e]);
  float* my = reinterpret_cast<float*>(lds + xf * C::PADN);
  LdsFft<M2, E, -1, WL, false, true, blue_split_pf(M2)>::run(v, my, nullptr, tw_f, tid);
  const float2* h = hp + (size_t)k1 * M2 + tid;
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = cmul(v[e], h[T * e]);
  LdsFft<M2, E, 1, WL, false, true, blue_split_pf(M2)>::run(v, my, nullptr, tw_i, tid);
  mul_roots<E, T, true>(v, lo, hi, (unsigned)k1, (unsigned)tid, m - 1, lo_bits);  // W_m^-(n2*k1)
#pragma unroll
  for (int e = 0; e < E; ++e) {
    pr[T * e] = v[e].x;
    pi[T * e] = v[e].y;
  }
}

template <int M1, int M2>
static hipError_t launch_blue_split_t(const BlueSplitArgs& a) {
  using G = BlueColCfg<M1>;
  using R = C2cThreads<M2>;
  static_assert(M2 % G::C == 0 && M1 % R::XF == 0, "split tiles");
  const int tiles = M2 / G::C;
  const unsigned cblocks = (unsigned)(a.batch * tiles);
  if (a.in_im == nullptr)
    hipLaunchKernelGGL((blue_col_fwd_kernel<M1, true>), dim3(cblocks), dim3(G::C * G::T), 0, a.stream, a.in_re,
                       a.in_im, a.ws_re, a.ws_im, a.chirp, a.tw1f, a.lo, a.hi, a.lo_bits, a.n, M2, tiles);
  else
    hipLaunchKernelGGL((blue_col_fwd_kernel<M1, false>), dim3(cblocks), dim3(G::C * G::T), 0, a.stream, a.in_re,
                       a.in_im, a.ws_re, a.ws_im, a.chirp, a.tw1f, a.lo, a.hi, a.lo_bits, a.n, M2, tiles);
  hipLaunchKernelGGL((blue_row_kernel<M2>), dim3((unsigned)(a.batch * M1 / R::XF)), dim3(R::THREADS), 0, a.stream,
                     a.ws_re, a.ws_im, a.hp, a.tw2f, a.tw2i, a.lo, a.hi, a.lo_bits, M1);
  hipLaunchKernelGGL((blue_col_inv_kernel<M1>), dim3(cblocks), dim3(G::C * G::T), 0, a.stream, a.ws_re, a.ws_im,
                     a.out_re, a.out_im, a.chirp, a.tw1i, a.n, M2, tiles, a.scale);
  return hipGetLastError();
}

hipError_t launch_bluestein_split(int m1, int m2, const BlueSplitArgs& a) {
  const long long key = (long long)m1 * 65536 + m2;
  switch (key) {
    case 128LL * 65536 + 128: return launch_blue_split_t<128, 128>(a);
    case 128LL * 65536 + 256: return launch_blue_split_t<128, 256>(a);
    case 256LL * 65536 + 256: return launch_blue_split_t<256, 256>(a);
    case 256LL * 65536 + 512: return launch_blue_split_t<256, 512>(a);
    case 512LL * 65536 + 512: return launch_blue_split_t<512, 512>(a);
    case 512LL * 65536 + 1024: return launch_blue_split_t<512, 1024>(a);
    case 1024LL * 65536 + 1024: return launch_blue_split_t<1024, 1024>(a);
    case 1024LL * 65536 + 2048: return launch_blue_split_t<1024, 2048>(a);
    case 2048LL * 65536 + 2048: return launch_blue_split_t<2048, 2048>(a);
    case 2048LL * 65536 + 4096: return launch_blue_split_t<2048, 4096>(a);
    case 4096LL * 65536 + 4096: return launch_blue_split_t<4096, 4096>(a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfa
