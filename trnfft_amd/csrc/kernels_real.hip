// Real-input forward (r2c) and real-output inverse (c2r) transforms of power-of-two length
// N = 2H, 4 <= N <= 32768, through one complex transform of half length.
//
// The reference computes rfft as a full length-N complex transform of (x, 0) and slices bins
// 0..N/2 (trnfft/api.py:38-46), and irfft by materialising the Hermitian-completed length-N
// spectrum and taking the real part of its inverse (trnfft/api.py:49-68).  Here:
//   r2c: z[m] = x[2m] + i x[2m+1] (the real row read as H float2), Z = FFT_H(z), then
//        X[k] = E[k] + W_N^k O[k],  E[k] = (Z[k] + conj Z[H-k]) / 2,  O[k] = (Z[k] - conj Z[H-k]) / 2i,
//        for k = 0..H-1, and X[H] = Re Z[0] - Im Z[0].
//   c2r: Z[k] = (X[k] + conj X[H-k]) + i W_N^-k (X[k] - conj X[H-k]), scaled by 1/N, for k < H
//        (Im X[0] and Im X[H] are dropped: they only feed the imaginary part the reference
//        discards), z = IFFT_H(Z) unnormalised, x[2m] = Re z[m], x[2m+1] = Im z[m].
// Half the HBM bytes of the complex formulation and half its arithmetic.
#include "kernels.h"

namespace tfa {

template <int H, int E_, int THR = 256>
struct RealCfg {
  static constexpr int E = E_;
  static constexpr int T = H / E;
  static constexpr int XF = T >= THR ? 1 : THR / T;  // transforms per workgroup
  static constexpr int THREADS = XF * T;
  static constexpr int PADR = lds_pad(H) + 1;  // room for bins 0..H
  // rows of H+1 bins with H <= 64: a store (r2c) or load (c2r) instruction would cover segments
  // of 64 bytes or less at odd alignment, one per row; the workgroup's XF rows of bins are one
  // contiguous run per plane, staged through LDS and moved as such
  static constexpr bool STAGE = H <= 64 && XF > 1;
  // r2c up to H = 256: the bins leave through the same staging as one run per plane, stored in
  // whole 128-byte lines (rows of H + 1 floats start off the line grid, so every row's own stores
  // split lines): rfft n = 256 9.5 -> 8.3 us, n = 512 8.5 -> 8.2, n = 128 7.7 -> 7.5 (4M samples);
  // n = 1024 and 2048 measured 1-3 % slower that way
  static constexpr bool STAGE_OUT = XF > 1 && H <= 256;
  // r2c at n = 32: the real rows come in the same way, one contiguous run per workgroup (rfft
  // n = 32 18.4 -> 15.5 us for 8M samples; n = 64 even, n = 128 9 % slower)
  static constexpr bool STAGE_IN = STAGE && H <= 16;
};

__device__ __forceinline__ float2 ld_stream2(const float2* p) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  const f2v r = __builtin_nontemporal_load(reinterpret_cast<const f2v*>(p));
  return make_float2(r.x, r.y);
}
__device__ __forceinline__ void st_stream2(float2* p, float2 v) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  f2v r;
  r.x = v.x;
  r.y = v.y;
  __builtin_nontemporal_store(r, reinterpret_cast<f2v*>(p));
}

// w[e] = base * W_{2E}^e (W = exp(DIR 2 pi i / 2E)): with base = W_N^tid this is W_N^(tid + T e)
// for N = 2 T E, so one table load per thread replaces E of them.
template <int E, int DIR, int I = 0>
struct TwRow {
  __device__ __forceinline__ static void fill(float2 (&w)[E], float2 base) {
    if constexpr (I < E) {
      w[I] = twiddle_const<I, 2 * E, DIR>(base);
      TwRow<E, DIR, I + 1>::fill(w, base);
    }
  }
};

// x: (batch, 2H) real rows; out: (batch, H+1) bins.  twr[k] = W_N^k = exp(-2 pi i k / N), k < H.
template <int H, bool TAIL, int E_ = real_epth(H, false), int THR = 256>
__global__ __launch_bounds__((RealCfg<H, E_, THR>::THREADS)) void r2c_kernel(
    const float* __restrict__ x, float* __restrict__ out_re, float* __restrict__ out_im,
    const float2* __restrict__ tw, const float2* __restrict__ twr, long long first, long long batch) {
  using C = RealCfg<H, E_, THR>;
  constexpr int E = C::E, T = C::T;
  constexpr bool WL = T <= 64;
  __shared__ float2 lds[C::XF * C::PADR];  // interleaved (re, im)
  __shared__ float2 stage[C::STAGE_OUT ? C::XF * (H + 1) : 1];  // the workgroup's bins, row after row
  const int tid = threadIdx.x % T;
  const int xf = threadIdx.x / T;
  const long long b0 = first + (long long)blockIdx.x * C::XF;
  const long long b = b0 + xf;
  const bool valid = !TAIL || b < batch;
  float2* m = lds + xf * C::PADR;
  float2 v[E];
  if constexpr (C::STAGE_IN) {
    // short rows: the workgroup's rows are one contiguous run of rows * 2H floats, loaded as such
    // (a thread's own float2 loads would cover 32-byte pieces of 16 rows per instruction) into the
    // bins' staging area, row r at r * (2H + 2) floats (an odd float2 pitch across rows)
    constexpr int NS = C::XF * 2 * H / C::THREADS;
    static_assert(NS * C::THREADS == C::XF * 2 * H, "the run is NS steps of the workgroup");
    const long long left = batch - b0;
    const int cnt = (TAIL ? (int)(left < C::XF ? left : C::XF) : C::XF) * 2 * H;
    const float* src0 = x + (size_t)b0 * (2 * H);
    float xs[NS];
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int i = (int)threadIdx.x + C::THREADS * u;
      xs[u] = ld_stream(src0 + (TAIL && i >= cnt ? cnt - 1 : i));
    }
    __builtin_amdgcn_sched_barrier(0);  // (else the scheduler pairs each load with its write)
    float* sf = reinterpret_cast<float*>(stage);
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int i = (int)threadIdx.x + C::THREADS * u;
      if (!TAIL || i < cnt) sf[(i / (2 * H)) * (2 * H + 2) + i % (2 * H)] = xs[u];
    }
    __syncthreads();
    // (rows past the batch read stale entries: transformed, never stored)
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = stage[xf * (H + 1) + tid + T * e];
    __syncthreads();  // the area takes the bins below
  } else {
    // a slot past the last row reads the last row (unconditional loads: under `valid ?` the
    // compiler waited for each load before issuing the next); its results are not stored
    const long long bl = valid ? b : batch - 1;
    const float2* src = reinterpret_cast<const float2*>(x + (size_t)bl * (2 * H)) + tid;
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = ld_stream2(src + T * e);
  }
  // the post-processing root W_N^tid, requested with the row (read where used, its load was
  // waited for after the transform)
  const float2 tw0 = twr[tid];
  LdsFft<H, E, -1, WL, false, true, real_pf(H)>::run(v, reinterpret_cast<float*>(m), nullptr, tw, tid);
#pragma unroll
  for (int e = 0; e < E; ++e) m[lds_pad(tid + T * e)] = v[e];
  exchange_sync<WL>();
  if (!C::STAGE_OUT && !valid) return;
  float* qr = out_re + (size_t)b * (H + 1) + tid;
  float* qi = out_im + (size_t)b * (H + 1) + tid;
  float2 wk[E];
  TwRow<E, -1>::fill(wk, tw0);  // W_N^k, k = tid + T e (9.8 -> 9.1 us against E table loads)
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = tid + T * e;
    const float2 z = m[lds_pad((H - k) & (H - 1))];
    const float2 a = v[e];
    const float2 c = make_float2(z.x, -z.y);  // conj Z[H-k]
    const float2 ev = make_float2(0.5f * (a.x + c.x), 0.5f * (a.y + c.y));
    const float2 od = make_float2(0.5f * (a.y - c.y), -0.5f * (a.x - c.x));  // (a - c) / 2i
    const float2 y = cadd(ev, cmul(wk[e], od));
    if constexpr (C::STAGE_OUT) {
      stage[xf * (H + 1) + k] = y;
    } else {
      st_stream(qr + T * e, y.x);
      st_stream(qi + T * e, y.y);
    }
  }
  if constexpr (C::STAGE_OUT) {
    if (tid == 0) stage[xf * (H + 1) + H] = make_float2(v[0].x - v[0].y, 0.0f);
    __syncthreads();
    // the rows b0 .. b0 + rows - 1 of bins are one contiguous run of rows * (H + 1) floats per
    // plane; lanes start early by the run's offset from a 128-byte line, so that every store
    // instruction of a full wavefront covers whole lines
    const long long left = batch - b0;
    const int rows = TAIL ? (int)(left < C::XF ? left : C::XF) : C::XF;
    const int count = rows * (H + 1);
    float* orr = out_re + (size_t)b0 * (H + 1);
    float* oii = out_im + (size_t)b0 * (H + 1);
    const int sh = (int)((reinterpret_cast<uintptr_t>(orr) >> 2) & 31);
    for (int i = (int)threadIdx.x - sh; i < count; i += C::THREADS) {
      if (i < 0) continue;
      const float2 y = stage[i];
      st_stream(orr + i, y.x);
      st_stream(oii + i, y.y);
    }
  } else if (tid == 0) {
    st_stream(qr + H, v[0].x - v[0].y);
    st_stream(qi + H, 0.0f);
  }
}

// in: (batch, H+1) bins; x: (batch, 2H) real rows.  tw: inverse LDS table of length H.
template <int H, bool TAIL, int E_ = real_epth(H, true), int THR = 256>
__global__ __launch_bounds__((RealCfg<H, E_, THR>::THREADS)) void c2r_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* __restrict__ x,
    const float2* __restrict__ tw, const float2* __restrict__ twr, long long first, long long batch, float scale) {
  using C = RealCfg<H, E_, THR>;
  constexpr int E = C::E, T = C::T;
  constexpr bool WL = T <= 64;
  __shared__ float2 lds[C::XF * C::PADR];  // interleaved (re, im)
  const int tid = threadIdx.x % T;
  const int xf = threadIdx.x / T;
  const long long b0 = first + (long long)blockIdx.x * C::XF;
  const long long b = b0 + xf;
  const bool valid = !TAIL || b < batch;
  float2* m = lds + xf * C::PADR;
  // tk: the post-processing roots W_N^k requested with the bins from H = 512 (irfft n = 1024
  // 8.02 -> 7.91 us, n = 2048 8.96 -> 8.83); read where used below that (n = 256 9.4 against 10.2
  // us requested early, n = 128 7.6 against 8.5)
  constexpr bool TKP = H >= 512;
  float2 a[E], tk[TKP ? E : 1];
  if constexpr (C::STAGE) {
    // the rows b0 .. b0 + rows - 1 of bins are one contiguous run of rows * (H + 1) floats per
    // plane: loaded as such into each row's LDS area (bin k of row r at r * PADR + lds_pad(k))
    const long long left = batch - b0;
    const int rows = TAIL ? (int)(left < C::XF ? left : C::XF) : C::XF;
    const int count = rows * (H + 1);
    const float* prr = in_re + (size_t)b0 * (H + 1);
    const float* pii = in_im + (size_t)b0 * (H + 1);
    // NS loads per thread, all issued before the first LDS write (a ragged tail rereads its
    // last bin)
    constexpr int NS = (C::XF * (H + 1) + C::THREADS - 1) / C::THREADS;
    float2 bs[NS];
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int i = (int)threadIdx.x + C::THREADS * u;
      const int ic = i < count ? i : count - 1;
      bs[u] = make_float2(ld_stream(prr + ic), ld_stream(pii + ic));
    }
    __builtin_amdgcn_sched_barrier(0);  // (else the scheduler pairs each load with its write)
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int i = (int)threadIdx.x + C::THREADS * u;
      if (i < count) {
        const int r = i / (H + 1), k = i - r * (H + 1);
        lds[r * C::PADR + lds_pad(k)] = bs[u];
      }
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) a[e] = valid ? m[lds_pad(tid + T * e)] : make_float2(0.0f, 0.0f);
    if (tid == 0) {
      m[lds_pad(H)].y = 0.0f;  // Im X[H] is never read
      a[0].y = 0.0f;           // Im X[0] drops out
    }
  } else {
    // a slot past the last row reads the last row (unconditional loads: under `valid ?` the
    // compiler waited for each load before issuing the next) and keeps zeros
    const long long bl = valid ? b : batch - 1;
    const float* pr = in_re + (size_t)bl * (H + 1) + tid;
    const float* pi = in_im + (size_t)bl * (H + 1) + tid;
#pragma unroll
    for (int e = 0; e < E; ++e) a[e] = make_float2(ld_stream(pr + T * e), ld_stream(pi + T * e));
    const float xh = ld_stream(in_re + (size_t)bl * (H + 1) + H);  // Re X[H] (every lane: one address)
    if constexpr (TKP) {
#pragma unroll
      for (int e = 0; e < E; ++e) tk[TKP ? e : 0] = twr[tid + T * e];
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (!valid) a[e] = make_float2(0.0f, 0.0f);
      m[lds_pad(tid + T * e)] = a[e];
    }
    // every lane of the row writes the same value (a store under `tid == 0` had the compiler sink
    // the load into that branch, one more memory round trip); Im X[H] is never read
    m[lds_pad(H)] = make_float2(valid ? xh : 0.0f, 0.0f);
    if (tid == 0) a[0].y = 0.0f;  // Im X[0] drops out
  }
  exchange_sync<WL>();
  float2 v[E];
  // (the table loads measured faster here than TwRow's derived twiddles: 8.2 vs 9.0 us)
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k = tid + T * e;
    const float2 z = m[lds_pad(H - k)];
    const float2 c = make_float2(z.x, k == 0 ? 0.0f : -z.y);  // conj X[H-k]
    const float2 sum = cadd(a[e], c);
    const float2 t = TKP ? tk[TKP ? e : 0] : twr[k];
    const float2 dif = cmul(csub(a[e], c), make_float2(t.x, -t.y));  // x W_N^-k
    v[e] = make_float2((sum.x - dif.y) * scale, (sum.y + dif.x) * scale);         // sum + i dif
  }
  exchange_sync<WL>();  // the transform below reuses this transform's LDS
  LdsFft<H, E, 1, WL, false, true, real_pf(H)>::run(v, reinterpret_cast<float*>(m), nullptr, tw, tid);
  if (!valid) return;
  float2* dst = reinterpret_cast<float2*>(x + (size_t)b * (2 * H)) + tid;
#pragma unroll
  for (int e = 0; e < E; ++e) st_stream2(dst + T * e, v[e]);
}

// Short rows (n = 2H = 8, 16): one thread per row, the half-length transform in registers (the
// in-register DFT).  A thread per row would touch one cache line per lane, so the workgroup's
// XS rows move between HBM and LDS as contiguous runs (rows of n reals, rows of H+1 bins); the
// input and output staging share the LDS area (a barrier between reading one and writing the
// other).
constexpr int kRealSmallRows = 256;

template <int H>
struct RealSmallCfg {
  static constexpr int XS = kRealSmallRows;
  static constexpr int PI = 2 * H + 1;  // real-row pitch in floats (odd: a column read hits distinct banks)
  static constexpr int PO = H + 1;      // bin-row pitch in float2 (odd for H >= 2)
  static constexpr int F2 = (XS * PI + 1) / 2 > XS * PO ? (XS * PI + 1) / 2 : XS * PO;  // float2 entries
};

template <int H, bool TAIL>
__global__ __launch_bounds__(kRealSmallRows) void r2c_small_kernel(
    const float* __restrict__ x, float* __restrict__ out_re, float* __restrict__ out_im,
    const float2* __restrict__ twr, long long first, long long batch) {
  using C = RealSmallCfg<H>;
  constexpr int N = 2 * H, XS = C::XS, PI = C::PI, PO = C::PO;
  __shared__ float2 lds[C::F2];
  float* lf = reinterpret_cast<float*>(lds);
  const long long r0 = first + (long long)blockIdx.x * XS;
  const int rows = TAIL ? (int)(batch - r0 < XS ? batch - r0 : XS) : XS;
  // N loads per thread, all issued before the first LDS write (a ragged tail rereads its last
  // sample)
  {
    const int cnt = rows * N;
    float xs[N];
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int i = (int)threadIdx.x + XS * u;
      xs[u] = ld_stream(x + (size_t)r0 * N + (TAIL && i >= cnt ? cnt - 1 : i));
    }
    __builtin_amdgcn_sched_barrier(0);  // (else the scheduler pairs each load with its write)
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int i = (int)threadIdx.x + XS * u;
      if (!TAIL || i < cnt) lf[(i / N) * PI + i % N] = xs[u];
    }
  }
  __syncthreads();
  float2 z[H];
  const float* row = lf + threadIdx.x * PI;  // rows past a ragged tail hold stale data, never stored
#pragma unroll
  for (int m = 0; m < H; ++m) z[m] = make_float2(row[2 * m], row[2 * m + 1]);
  __syncthreads();  // the staging area is rewritten with bins below
  Dft<H, -1>::run(z);
  float2* out = lds + threadIdx.x * PO;
#pragma unroll
  for (int k = 0; k < H; ++k) {
    const float2 a = z[k], zc = z[(H - k) & (H - 1)];
    const float2 c = make_float2(zc.x, -zc.y);  // conj Z[H-k]
    const float2 ev = make_float2(0.5f * (a.x + c.x), 0.5f * (a.y + c.y));
    const float2 od = make_float2(0.5f * (a.y - c.y), -0.5f * (a.x - c.x));  // (a - c) / 2i
    out[k] = cadd(ev, cmul(twr[k], od));
  }
  out[H] = make_float2(z[0].x - z[0].y, 0.0f);
  __syncthreads();
  for (int i = threadIdx.x; i < rows * PO; i += XS) {
    const float2 y = lds[(i / PO) * PO + i % PO];
    st_stream(out_re + (size_t)r0 * PO + i, y.x);
    st_stream(out_im + (size_t)r0 * PO + i, y.y);
  }
}

template <int H, bool TAIL>
__global__ __launch_bounds__(kRealSmallRows) void c2r_small_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* __restrict__ x,
    const float2* __restrict__ twr, long long first, long long batch, float scale) {
  using C = RealSmallCfg<H>;
  constexpr int N = 2 * H, XS = C::XS, PI = C::PI, PO = C::PO;
  __shared__ float2 lds[C::F2];
  float* lf = reinterpret_cast<float*>(lds);
  const long long r0 = first + (long long)blockIdx.x * XS;
  const int rows = TAIL ? (int)(batch - r0 < XS ? batch - r0 : XS) : XS;
  // PO bins per thread, all loads issued before the first LDS write (a ragged tail rereads its
  // last bin)
  {
    const int cnt = rows * PO;
    float2 bs[PO];
#pragma unroll
    for (int u = 0; u < PO; ++u) {
      const int i = (int)threadIdx.x + XS * u;
      const size_t o = (size_t)r0 * PO + (TAIL && i >= cnt ? cnt - 1 : i);
      bs[u] = make_float2(ld_stream(in_re + o), ld_stream(in_im + o));
    }
    __builtin_amdgcn_sched_barrier(0);  // (else the scheduler pairs each load with its write)
#pragma unroll
    for (int u = 0; u < PO; ++u) {
      const int i = (int)threadIdx.x + XS * u;
      if (!TAIL || i < cnt) lds[i] = bs[u];
    }
  }
  __syncthreads();
  float2 a[H + 1];
  const float2* bins = lds + threadIdx.x * PO;
#pragma unroll
  for (int k = 0; k <= H; ++k) a[k] = bins[k];
  __syncthreads();  // the staging area is rewritten with samples below
  a[0].y = 0.0f;  // Im X[0] and Im X[H] only feed the imaginary part the reference discards
  a[H].y = 0.0f;
  float2 z[H];
#pragma unroll
  for (int k = 0; k < H; ++k) {
    const float2 c = make_float2(a[H - k].x, -a[H - k].y);  // conj X[H-k]
    const float2 sum = cadd(a[k], c);
    const float2 dif = cmul(csub(a[k], c), make_float2(twr[k].x, -twr[k].y));  // x W_N^-k
    z[k] = make_float2((sum.x - dif.y) * scale, (sum.y + dif.x) * scale);        // sum + i dif
  }
  Dft<H, 1>::run(z);
  float* row = lf + threadIdx.x * PI;
#pragma unroll
  for (int m = 0; m < H; ++m) {
    row[2 * m] = z[m].x;
    row[2 * m + 1] = z[m].y;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < rows * N; i += XS) st_stream(x + (size_t)r0 * N + i, lf[(i / N) * PI + i % N]);
}

template <int H>
static hipError_t launch_real_small(const RealArgs& a) {
  // ragged batches: one launch of the guarded variant (a separate one-workgroup tail launch
  // measured ~3.5 us extra)
  const long long blocks = (a.batch + kRealSmallRows - 1) / kRealSmallRows;
  const bool ragged = blocks * kRealSmallRows != a.batch;
  if (a.inverse) {
    if (!ragged)
      hipLaunchKernelGGL((c2r_small_kernel<H, false>), dim3((unsigned)blocks), dim3(kRealSmallRows), 0, a.stream,
                         a.in_re, a.in_im, a.out_re, a.twr, 0LL, a.batch, a.scale);
    else
      hipLaunchKernelGGL((c2r_small_kernel<H, true>), dim3((unsigned)blocks), dim3(kRealSmallRows), 0, a.stream,
                         a.in_re, a.in_im, a.out_re, a.twr, 0LL, a.batch, a.scale);
  } else {
    if (!ragged)
      hipLaunchKernelGGL((r2c_small_kernel<H, false>), dim3((unsigned)blocks), dim3(kRealSmallRows), 0, a.stream,
                         a.in_re, a.out_re, a.out_im, a.twr, 0LL, a.batch);
    else
      hipLaunchKernelGGL((r2c_small_kernel<H, true>), dim3((unsigned)blocks), dim3(kRealSmallRows), 0, a.stream,
                         a.in_re, a.out_re, a.out_im, a.twr, 0LL, a.batch);
  }
  return hipGetLastError();
}

template <int H>
static hipError_t launch_real_h(const RealArgs& a) {
  // the short-row kernels for n = 8 and 16; n = 4 and n >= 32 measured faster on the LDS kernels
  // (n = 4: 8.6 vs 11.2 us for 4M samples; n = 32 with its bins staged through LDS: r2c 17.0 ->
  // 10.6 us, c2r 12.4 -> 8.7, 1000 rows 11.3 -> 4.7; n = 16 is even there, n = 8 slower)
  if constexpr (H >= 4 && H <= 8) {
    return launch_real_small<H>(a);
  } else {
    // ragged batches: one launch of the guarded variant
    if (a.inverse) {
      using C = RealCfg<H, real_epth(H, true)>;
      const long long blocks = (a.batch + C::XF - 1) / C::XF;
      if (blocks * C::XF == a.batch)
        hipLaunchKernelGGL((c2r_kernel<H, false>), dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream, a.in_re,
                           a.in_im, a.out_re, a.tw, a.twr, 0LL, a.batch, a.scale);
      else
        hipLaunchKernelGGL((c2r_kernel<H, true>), dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream, a.in_re,
                           a.in_im, a.out_re, a.tw, a.twr, 0LL, a.batch, a.scale);
    } else {
      using C = RealCfg<H, real_epth(H, false)>;
      const long long blocks = (a.batch + C::XF - 1) / C::XF;
      if (blocks * C::XF == a.batch)
        hipLaunchKernelGGL((r2c_kernel<H, false>), dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream, a.in_re,
                           a.out_re, a.out_im, a.tw, a.twr, 0LL, a.batch);
      else
        hipLaunchKernelGGL((r2c_kernel<H, true>), dim3((unsigned)blocks), dim3(C::THREADS), 0, a.stream, a.in_re,
                           a.out_re, a.out_im, a.tw, a.twr, 0LL, a.batch);
    }
    return hipGetLastError();
  }
}

hipError_t launch_real(int n, const RealArgs& a) {
  switch (n) {
    case 4: return launch_real_h<2>(a);
    case 8: return launch_real_h<4>(a);
    case 16: return launch_real_h<8>(a);
    case 32: return launch_real_h<16>(a);
    case 64: return launch_real_h<32>(a);
    case 128: return launch_real_h<64>(a);
    case 256: return launch_real_h<128>(a);
    case 512: return launch_real_h<256>(a);
    case 1024: return launch_real_h<512>(a);
    case 2048: return launch_real_h<1024>(a);
    case 4096: return launch_real_h<2048>(a);
    case 8192: return launch_real_h<4096>(a);
    case 16384: return launch_real_h<8192>(a);
    case 32768: return launch_real_h<16384>(a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfa
