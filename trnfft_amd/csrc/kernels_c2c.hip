// Batched power-of-two complex-to-complex FFT kernels.
//
//  * c2c_lds_kernel: one launch per batch; each transform of length N <= 16384 stays in
//    registers + LDS for all its passes (replaces the reference's per-stage launches,
//    trnfft/fft_core.py:53-117 on CPU and :1063-1238 on the NKI path).
//  * strided_kernel: transform along a non-contiguous axis (element stride S), C adjacent
//    columns per workgroup; replaces the transpose copies of trnfft/api.py:496-516 for fftn/fft2.
//  * four-step (fourstep_col_kernel + fourstep_row_kernel): N = N1*N2 > 16384 in two HBM passes
//    (column FFTs with the W_N^{n2*k1} twiddle, written in a blocked layout that the row pass
//    reads contiguously; row FFTs stored to the transposed output with whole-line segments).
//    This is the single-GPU form of the reference's row-column decomposition,
//    trnfft/nki/multicore.py:151-219.
#include "kernels.h"

namespace tfa {

// ---------------------------------------------------------------------------------------------
// LDS-resident batched transform
// ---------------------------------------------------------------------------------------------
// TAIL = false: every transform slot of the grid is inside the batch (no guards at all; the
// guard-free instruction stream measured fastest).  TAIL = true: the launch for a ragged batch,
// whose slots past the batch end neither load nor store (one launch instead of a full-block
// launch plus a one-workgroup tail launch: 4095 x 1024 18.2 -> 13.3 us).
template <int N, int DIR, bool REAL_IN, bool TAIL, int E_ = c2c_epth(N), int THR = c2c_threads(N)>
__global__ __launch_bounds__((C2cThreads<N, E_, THR>::THREADS)) void c2c_lds_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re,
    float* out_im, const float2* __restrict__ tw, long long first, long long batch, float scale) {
  using C = C2cThreads<N, E_, THR>;
  constexpr int E = C::E, T = C::T;
  // interleaved (re, im) exchange, or two planes, in the same LDS bytes
  constexpr bool IL = c2c_il(N);
  __shared__ float2 lds[C::XF * C::PADN];
  const int tid = threadIdx.x & (T - 1);
  const int xf = threadIdx.x / T;
  const long long b = first + (long long)blockIdx.x * C::XF + xf;
  const bool valid = !TAIL || b < batch;
  const size_t base = (size_t)b * N;
  // one base pointer per plane; element e is at a compile-time offset T*e (immediate offsets)
  const float* pr = in_re + base + tid;
  const float* pi = REAL_IN ? nullptr : in_im + base + tid;
  // inverse: the 1/n factor is applied to the input (exact for power-of-two n), keeping the
  // store sequence free of multiplies
  const float sc = DIR < 0 ? 1.0f : scale;
  float2 v[E];
  if (valid) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float xr = ld_stream(pr + T * e);
      const float xi = REAL_IN ? 0.0f : ld_stream(pi + T * e);
      v[e] = DIR < 0 ? make_float2(xr, xi) : make_float2(xr * sc, xi * sc);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = make_float2(0.0f, 0.0f);
  }
  constexpr bool PF = c2c_pf(N);
  if constexpr (IL) {
    LdsFft<N, E, DIR, (T <= 64), false, true, PF>::run(v, reinterpret_cast<float*>(lds + xf * C::PADN), nullptr, tw,
                                                      tid);
  } else {
    float* planes = reinterpret_cast<float*>(lds);
    LdsFft<N, E, DIR, (T <= 64), false, false, PF>::run(v, planes + xf * C::PADN, planes + (C::XF + xf) * C::PADN, tw,
                                                       tid);
  }
  if (valid) {
    float* qr = out_re + base + tid;
    float* qi = out_im + base + tid;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      st_stream(qr + T * e, v[e].x);
      st_stream(qi + T * e, v[e].y);
    }
  }
}

// Short transforms (2 <= N <= 64): a few threads per row (one up to N = 16, the whole transform
// an in-register DFT; N / c2c_epth(N) above, exchanging through the row's own LDS area inside a
// wavefront).  Threads that each load their own row segment would touch one cache line per
// lane (N <= 16) or half a line (N = 32, 64), so the workgroup's XS rows move between HBM and
// LDS as one contiguous run per plane: every global access instruction covers 64 consecutive
// floats (4M elements: N = 16 169 -> 15 us, N = 32 33 -> 12 us).
template <int N>
struct C2cSmallCfg {
  static constexpr int TPR = N <= 8 ? 1 : N / c2c_epth(N);  // threads per row
  static constexpr int XS = TPR <= 4 ? 256 : 1024 / TPR;     // rows per workgroup
  static constexpr int E = N / TPR;
  static constexpr int THREADS = XS * TPR;
  // row pitch in float2: odd, and room for the exchange's padded indexing when TPR > 1
  static constexpr int P = TPR == 1 ? N + 1 : lds_pad(N) + 1;
  __device__ static constexpr int idx(int j) { return TPR == 1 ? j : lds_pad(j); }
};

template <int N, int DIR, bool REAL_IN, bool TAIL>
__global__ __launch_bounds__(C2cSmallCfg<N>::THREADS) void c2c_small_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re, float* out_im,
    const float2* __restrict__ tw, long long first, long long batch, float scale) {
  using C = C2cSmallCfg<N>;
  constexpr int XS = C::XS, P = C::P, TPR = C::TPR, E = C::E, THREADS = C::THREADS;
  static_assert(XS * N == THREADS * E, "the tile's floats per plane are E steps of THREADS");
  __shared__ float2 lds[XS * P];
  const long long r0 = first + (long long)blockIdx.x * XS;
  const int count = TAIL ? (int)(batch - r0 < XS ? batch - r0 : XS) * N : XS * N;  // floats per plane
  const size_t g0 = (size_t)r0 * N;
  const float sc = DIR < 0 ? 1.0f : scale;  // inverse: 1/n applied on input (exact for powers of two)
  // E loads per thread, all issued before the first LDS write (a load-then-store loop waits out
  // the memory latency once per step); a ragged tail reads its last element again
  float xr[E], xi[E];
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int i = (int)threadIdx.x + THREADS * u;
    const int ic = TAIL && i >= count ? count - 1 : i;
    xr[u] = ld_stream(in_re + g0 + ic);
    xi[u] = REAL_IN ? 0.0f : ld_stream(in_im + g0 + ic);
  }
  __builtin_amdgcn_sched_barrier(0);  // (else the scheduler pairs each load with its write)
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int i = (int)threadIdx.x + THREADS * u;
    if (!TAIL || i < count) lds[(i / N) * P + C::idx(i % N)] = make_float2(xr[u] * sc, xi[u] * sc);
  }
  __syncthreads();
  const int tid = threadIdx.x % TPR;
  float2* row = lds + (threadIdx.x / TPR) * P;  // rows past a ragged tail hold stale data, never stored
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = row[C::idx(tid + TPR * e)];
  if constexpr (TPR == 1) {
    Dft<N, DIR>::run(v);
  } else {
    exchange_sync<true>();  // the row's area becomes its exchange area (one wavefront per row group)
    LdsFft<N, E, DIR, true, false, true>::run(v, reinterpret_cast<float*>(row), nullptr, tw, tid);
    exchange_sync<true>();
  }
#pragma unroll
  for (int e = 0; e < E; ++e) row[C::idx(tid + TPR * e)] = v[e];
  __syncthreads();
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int i = (int)threadIdx.x + THREADS * u;
    if (!TAIL || i < count) {
      const float2 y = lds[(i / N) * P + C::idx(i % N)];
      st_stream(out_re + g0 + i, y.x);
      st_stream(out_im + g0 + i, y.y);
    }
  }
}

template <int N, int DIR, bool REAL_IN>
static hipError_t launch_c2c_small_t(const C2cArgs& a) {
  constexpr int THREADS = C2cSmallCfg<N>::THREADS, XS = C2cSmallCfg<N>::XS;
  const long long blocks = (a.batch + XS - 1) / XS;
  if (blocks * XS == a.batch)
    hipLaunchKernelGGL((c2c_small_kernel<N, DIR, REAL_IN, false>), dim3((unsigned)blocks), dim3(THREADS), 0,
                       a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw, 0LL, a.batch, a.scale);
  else  // ragged batch: one launch whose slots past the end neither load nor store
    hipLaunchKernelGGL((c2c_small_kernel<N, DIR, REAL_IN, true>), dim3((unsigned)blocks), dim3(THREADS), 0,
                       a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw, 0LL, a.batch, a.scale);
  return hipGetLastError();
}

template <int N, int DIR, bool REAL_IN>
static hipError_t launch_c2c_lds_t(const C2cArgs& a) {
  if constexpr (N >= 2 && N <= 64) {
    return launch_c2c_small_t<N, DIR, REAL_IN>(a);
  } else {
    using C = C2cThreads<N>;
    const long long blocks = (a.batch + C::XF - 1) / C::XF;
    if (blocks * C::XF == a.batch)
      hipLaunchKernelGGL((c2c_lds_kernel<N, DIR, REAL_IN, false>), dim3((unsigned)blocks), dim3(C::THREADS), 0,
                         a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw, 0LL, a.batch, a.scale);
    else  // ragged batch: one launch whose slots past the end neither load nor store
      hipLaunchKernelGGL((c2c_lds_kernel<N, DIR, REAL_IN, true>), dim3((unsigned)blocks), dim3(C::THREADS), 0,
                         a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw, 0LL, a.batch, a.scale);
    return hipGetLastError();
  }
}

template <int N>
static hipError_t launch_c2c_lds_n(const C2cArgs& a) {
  const bool real_in = a.in_im == nullptr;
  if (a.dir < 0)
    return real_in ? launch_c2c_lds_t<N, -1, true>(a) : launch_c2c_lds_t<N, -1, false>(a);
  return real_in ? launch_c2c_lds_t<N, 1, true>(a) : launch_c2c_lds_t<N, 1, false>(a);
}

hipError_t launch_c2c_lds(int n, const C2cArgs& a) {
  switch (n) {
    case 1: return launch_c2c_lds_n<1>(a);
    case 2: return launch_c2c_lds_n<2>(a);
    case 4: return launch_c2c_lds_n<4>(a);
    case 8: return launch_c2c_lds_n<8>(a);
    case 16: return launch_c2c_lds_n<16>(a);
    case 32: return launch_c2c_lds_n<32>(a);
    case 64: return launch_c2c_lds_n<64>(a);
    case 128: return launch_c2c_lds_n<128>(a);
    case 256: return launch_c2c_lds_n<256>(a);
    case 512: return launch_c2c_lds_n<512>(a);
    case 1024: return launch_c2c_lds_n<1024>(a);
    case 2048: return launch_c2c_lds_n<2048>(a);
    case 4096: return launch_c2c_lds_n<4096>(a);
    case 8192: return launch_c2c_lds_n<8192>(a);
    case 16384: return launch_c2c_lds_n<16384>(a);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------------------------
// Strided-axis transform: x viewed as (outer, N1, S) row-major; transform along the N1 axis
// (element stride S) for every (outer, column) pair.  One workgroup = C adjacent columns of one
// outer block, so each load/store instruction covers C consecutive floats.
// ---------------------------------------------------------------------------------------------
template <int N1, int DIR, bool REAL_IN, int C = fourstep_tile(N1)>
__global__ __launch_bounds__(C * (N1 / lds_epth(N1))) void strided_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re, float* out_im,
    const float2* __restrict__ tw, long long stride, int tiles_per_block, float scale) {
  constexpr int E = lds_epth(N1), T = N1 / E;
  constexpr int PADN = lds_pad(N1) + 1;
  // interleaved (re, im) exchange except at 4096 (two planes measured 3.5 % faster there)
  constexpr bool IL = N1 != 4096;
  __shared__ float2 lds[C * PADN];
  const int c = threadIdx.x % C;  // column within tile (fast across lanes: coalesced)
  const int t = threadIdx.x / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_block;
  const long long col = (tile % tiles_per_block) * C + c;
  const bool valid = col < stride;
  const size_t base = (size_t)b * N1 * stride + col;
  // a column past the last reads the last column (unconditional loads: under `valid ?` the
  // compiler waited for each load before issuing the next); its results are not stored
  const size_t lbase = valid ? base : base - (size_t)(col - (stride - 1));

  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = lbase + (size_t)(t + T * e) * stride;
    v[e] = make_float2(ld_stream(in_re + i), REAL_IN ? 0.0f : ld_stream(in_im + i));
  }
  if constexpr (IL) {
    LdsFft<N1, E, DIR, false, false, true>::run(v, reinterpret_cast<float*>(lds + c * PADN), nullptr, tw, t);
  } else {
    float* planes = reinterpret_cast<float*>(lds);
    LdsFft<N1, E, DIR, false>::run(v, planes + c * PADN, planes + (C + c) * PADN, tw, t);
  }
  if (!valid) return;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float2 y = cscale(v[e], scale);
    const size_t i = base + (size_t)(t + T * e) * stride;
    if constexpr (C * 4 < 128) {
      // row segments shorter than a cache line: plain stores, so L2 merges the partial lines
      // of neighbouring workgroups before they reach HBM (measured 1.1x faster at N1 = 1024)
      out_re[i] = y.x;
      out_im[i] = y.y;
    } else {
      st_stream(out_re + i, y.x);
      st_stream(out_im + i, y.y);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Four-step: x viewed as (N1 rows) x (N2 columns), n = N2*n1 + n2, k = k1 + N1*k2.
//   pass 1 (fourstep_col_kernel): DFT over n1 of TILE adjacent columns n2, times W_N^(n2*k1),
//     written to the workspace in the blocked layout tmp[kb][n2][kk] with k1 = kb*CK + kk and CK
//     the pass-2 tile, so the tile's output is N1/CK contiguous runs of TILE*CK floats;
//   pass 2 (fourstep_row_kernel): DFT over n2 of the CK rows k1 = kb*CK + r, read as one
//     contiguous CK*N2 run, stored to X[k1 + N1*k2] with CK consecutive k1 per store.
// With 32-transform tiles (lengths up to 1024) every HBM side of both passes moves whole 128-byte
// lines; 2048 and 4096 use 16 and 8 transforms per tile (the LDS holds no more).
// ---------------------------------------------------------------------------------------------
// TILE_ = 0: the wide tile, 1024 threads (32 transforms up to L = 1024, 16 at 2048, 8 at 4096).
// A narrower tile (TILE_ = kFourStepNarrow) spreads a small batch over more workgroups.
template <int L, int TILE_ = 0>
struct FourStepCfg {
  static constexpr int E = fourstep_epth(L);
  static constexpr int T = L / E;
  static constexpr int TILE = TILE_ ? TILE_ : 1024 / T;
  static constexpr int THREADS = TILE * T;
  static constexpr int PADN = lds_pad(L) + 1;
  // both planes (interleaved) in LDS when they fit in half of it (two workgroups per CU), else
  // the real and imaginary planes take turns (L = 512: 64 x 2^18 141 -> 133 us)
  static constexpr bool SPLIT = 2LL * TILE * PADN * 4 > kLdsBytes / 2;
  static_assert(THREADS <= 1024 && (SPLIT ? 1LL : 2LL) * TILE * PADN * 4 <= kLdsBytes, "four-step tile");
};
constexpr int kFourStepNarrow = 8;

// Entries of the W_N^lo / W_N^hi tables the column pass can stage in LDS without lowering its
// occupancy: the LDS its tile leaves free within its share of the CU (one, two, ... workgroups).
template <int N1, int TILE_>
constexpr int fourstep_twl_cap() {
  using Cfg = FourStepCfg<N1, TILE_>;
  constexpr long long tile = (Cfg::SPLIT ? 1LL : 2LL) * Cfg::TILE * Cfg::PADN * 4;
  constexpr long long per_cu = kLdsBytes / tile;  // workgroups per CU by LDS
  return per_cu > 0 ? (int)((kLdsBytes / per_cu - tile) / 8) : 0;
}

// TWL: the W_N^lo and W_N^hi tables are staged in LDS at the start (their global loads overlap the
// tile's), so the twiddle between the passes reads LDS instead of waiting out one L2 round trip per
// group of factors.
template <int N1, int DIR, bool REAL_IN, int CK, int TILE_ = 0, bool TWL = false>
__global__ __launch_bounds__((FourStepCfg<N1, TILE_>::THREADS)) void fourstep_col_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, const float2* __restrict__ tw_lo,
    const float2* __restrict__ tw_hi, long long stride, int tiles_per_block, int lo_bits, unsigned nmask) {
  using Cfg = FourStepCfg<N1, TILE_>;
  constexpr int C = Cfg::TILE, E = Cfg::E, T = Cfg::T, THREADS = Cfg::THREADS, PADN = Cfg::PADN;
  constexpr bool SPLIT = Cfg::SPLIT;
  constexpr int TF = E < 4 ? E : 4;  // twiddle factor group
  constexpr int CAP = TWL ? fourstep_twl_cap<N1, TILE_>() : 1;
  // split planes take turns through one float plane; otherwise interleaved (re, im) entries
  __shared__ float2 lds[SPLIT ? (C * PADN + 1) / 2 : C * PADN];
  __shared__ float2 twt[CAP > 0 ? CAP : 1];  // TWL: W^lo entries, then W^hi
  float* lre = reinterpret_cast<float*>(lds);
  const int nlo = 1 << lo_bits;
  if constexpr (TWL) {
    const int ntw = nlo + (int)((nmask >> lo_bits) + 1);
    for (int i = threadIdx.x; i < ntw; i += THREADS) twt[i] = i < nlo ? tw_lo[i] : tw_hi[i - nlo];
  }
  const int c = threadIdx.x % C;  // column within the tile (fast across lanes: whole lines)
  const int t = threadIdx.x / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_block;
  const long long col0 = (tile % tiles_per_block) * C;
  const unsigned col = (unsigned)(col0 + c);
  // per-thread base plus a workgroup-uniform offset per element (no per-element index math)
  const size_t base = (size_t)b * N1 * stride + col + (size_t)t * stride;
  const size_t step = (size_t)T * stride;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = base + e * step;
    v[e] = make_float2(ld_stream(in_re + i), REAL_IN ? 0.0f : ld_stream(in_im + i));
  }
  if constexpr (SPLIT)
    LdsFft<N1, E, DIR, false, true>::run(v, lre + c * PADN, nullptr, tw, t);
  else
    LdsFft<N1, E, DIR, false, false, true>::run(v, reinterpret_cast<float*>(lds + c * PADN), nullptr, tw, t);

  // W_N^(col*k1) for k1 = t + T*(TF*a + q): W^(col*(t + T*TF*a)) * W^(col*T*q), each root read as
  // W^lo * W^hi from the two small tables (TF-1 + E/TF table pairs per thread instead of E);
  // the scheduling barrier keeps one group's loads in flight at a time (register pressure)
  const unsigned lomask = (1u << lo_bits) - 1;
  // (the staged tables were written before the transform, whose exchanges are barriers)
  const float2* tlo = TWL ? twt : tw_lo;
  const float2* thi = TWL ? twt + nlo : tw_hi;
  float2 q[TF];
#pragma unroll
  for (int j = 1; j < TF; ++j) {
    const unsigned m = (col * (unsigned)(T * j)) & nmask;
    q[j] = cmul(tlo[m & lomask], thi[m >> lo_bits]);
  }
#pragma unroll
  for (int a = 0; a < E / TF; ++a) {
    const unsigned m = (col * (unsigned)(t + T * TF * a)) & nmask;
    const float2 p = cmul(tlo[m & lomask], thi[m >> lo_bits]);
    v[TF * a] = cmul(v[TF * a], p);
#pragma unroll
    for (int j = 1; j < TF; ++j) v[TF * a + j] = cmul(v[TF * a + j], cmul(p, q[j]));
    __builtin_amdgcn_sched_barrier(0);
  }

  // blocked store through LDS: linear position w of a run holds (column w / CK, kk = w % CK)
  const size_t obase = (size_t)b * N1 * stride + (size_t)col0 * CK;
  __syncthreads();  // every lane is past the transform's last LDS read
#pragma unroll
  for (int plane = 0; plane < (SPLIT ? 2 : 1); ++plane) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int idx = c * PADN + (T % 16 == 0 ? lds_pad(t) + e * (T + T / 16) : lds_pad(t + T * e));
      if constexpr (SPLIT) {
        lre[idx] = plane ? v[e].y : v[e].x;
      } else {
        lds[idx] = v[e];
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < E; ++i) {
      // thread x stores position w = x % RUN of run kb = x / RUN + RPI * i (RUN = C*CK floats)
      constexpr int RUN = C * CK, RPI = THREADS / RUN;
      const int w = threadIdx.x % RUN, kk = w % CK, kb = threadIdx.x / RUN + RPI * i;
      const int idx = (w / CK) * PADN +
                      (CK % 16 == 0 ? lds_pad(kk) + kb * (CK + CK / 16) : lds_pad(kb * CK + kk));
      const size_t o = obase + (size_t)(threadIdx.x / RUN) * stride * CK + w + (size_t)(RPI * i) * stride * CK;
      // plain stores (and plain loads in the row pass): the workspace is written and read once
      // within one transform and stays in the Infinity Cache between the passes when it fits
      // (16 x 2^20: 128 MB; C4b 121.9 -> 106.4 us against streaming accesses)
      if constexpr (SPLIT) {
        (plane ? out_im : out_re)[o] = lre[idx];
      } else {
        const float2 y = lds[idx];
        out_re[o] = y.x;
        out_im[o] = y.y;
      }
    }
    if (SPLIT && plane == 0) __syncthreads();
  }
}

// TWL: the transform's twiddle table is staged in LDS at the start (where it fits beside the tile
// at the same occupancy), so its table reads do not wait on L2.
template <int N2, int DIR, int TILE_ = 0, bool TWL = false>
__global__ __launch_bounds__((FourStepCfg<N2, TILE_>::THREADS)) void fourstep_row_kernel(
    const float* __restrict__ t_re, const float* __restrict__ t_im, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, int n1_len, float scale) {
  using Cfg = FourStepCfg<N2, TILE_>;
  constexpr int CK = Cfg::TILE, E = Cfg::E, T = Cfg::T, PADN = Cfg::PADN;
  constexpr bool SPLIT = Cfg::SPLIT;
  constexpr int NTW = make_shape(N2, E).twoff[make_shape(N2, E).npass];
  __shared__ float2 lds[SPLIT ? (CK * PADN + 1) / 2 : CK * PADN];
  __shared__ __attribute__((aligned(16))) float2 twt[TWL && NTW > 0 ? NTW : 2];
  float* lre = reinterpret_cast<float*>(lds);
  if constexpr (TWL) {
    // (read after the transform's first exchange, a barrier)
    for (int i = threadIdx.x; i < NTW; i += Cfg::THREADS) twt[i] = tw[i];
  }
  const float2* twx = TWL ? twt : tw;
  const int r = threadIdx.x % CK;  // row within the tile (fast across lanes)
  const int t = threadIdx.x / CK;
  const int tiles_per_b = n1_len / CK;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_b;
  const int kb = (int)(tile % tiles_per_b);
  const size_t N = (size_t)n1_len * N2;
  const size_t ibase = (size_t)b * N + (size_t)kb * N2 * CK + r + (size_t)t * CK;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = ibase + (size_t)e * (T * CK);
    v[e] = make_float2(t_re[i], t_im[i]);
  }
  if constexpr (SPLIT)
    LdsFft<N2, E, DIR, false, true>::run(v, lre + r * PADN, nullptr, twx, t);
  else
    LdsFft<N2, E, DIR, false, false, true>::run(v, reinterpret_cast<float*>(lds + r * PADN), nullptr, twx, t);
  const size_t obase = (size_t)b * N + (size_t)kb * CK + r + (size_t)t * n1_len;
  const size_t ostep = (size_t)T * n1_len;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t o = obase + e * ostep;
    if constexpr (CK * 4 < 128) {  // sub-line segments: plain stores (L2 merges them)
      out_re[o] = v[e].x * scale;
      out_im[o] = v[e].y * scale;
    } else {
      st_stream(out_re + o, v[e].x * scale);
      st_stream(out_im + o, v[e].y * scale);
    }
  }
}

// Strided transform with few columns (stride <= C/2): the column tile of strided_kernel would be
// mostly idle and its row segments a few floats long.  Here a workgroup takes G = C / stride
// whole (N1 x stride) blocks, contiguous in memory: they are read and written as one run per
// plane and transposed through LDS (column g*stride + col of the tile at region c*PADN, the
// transform's own exchange area, entry j at lds_pad(j)).  The transform prefetches each next
// pass's twiddles (n = 128 over 3 columns: 33.8 -> 31.9 us).
template <int N1, int DIR, bool REAL_IN, int C = fourstep_tile(N1)>
__global__ __launch_bounds__(C * (N1 / lds_epth(N1))) void strided_small_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, long long outer, int stride, int groups,
    float scale) {
  constexpr int E = lds_epth(N1), T = N1 / E, THREADS = C * T;
  constexpr int PADN = lds_pad(N1) + 1;
  __shared__ float2 lds[C * PADN];
  const long long o0 = (long long)blockIdx.x * groups;  // first block of the tile
  const int ng = (int)(outer - o0 < groups ? outer - o0 : groups);
  const int blk = N1 * stride;    // floats per block
  const int count = ng * blk;     // floats per plane in the tile (< 2^24: C * N1 <= 2^18)
  const size_t g0 = (size_t)o0 * blk;
  const float rs = 1.0f / (float)stride;
  const float rb = 1.0f / (float)blk;
  for (int i = threadIdx.x; i < count; i += THREADS) {
    int rem, col;
    const int g = divmod_small(i, blk, rb, rem);
    const int j = divmod_small(rem, stride, rs, col);
    const float xr = ld_stream(in_re + g0 + i);
    const float xi = REAL_IN ? 0.0f : ld_stream(in_im + g0 + i);
    lds[(g * stride + col) * PADN + lds_pad(j)] = make_float2(xr, xi);
  }
  __syncthreads();
  const int c = threadIdx.x % C, t = threadIdx.x / C;  // columns past the tile's ng*stride: stale, never stored
  float2* base = lds + c * PADN;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = base[lds_pad(t + T * e)];
  __syncthreads();  // the column area becomes the transform's exchange area
  LdsFft<N1, E, DIR, false, false, true, true>::run(v, reinterpret_cast<float*>(base), nullptr, tw, t);
  __syncthreads();
#pragma unroll
  for (int e = 0; e < E; ++e) base[lds_pad(t + T * e)] = cscale(v[e], scale);
  __syncthreads();
  for (int i = threadIdx.x; i < count; i += THREADS) {
    int rem, col;
    const int g = divmod_small(i, blk, rb, rem);
    const int j = divmod_small(rem, stride, rs, col);
    const float2 y = lds[(g * stride + col) * PADN + lds_pad(j)];
    st_stream(out_re + g0 + i, y.x);
    st_stream(out_im + g0 + i, y.y);
  }
}

template <int N1, int DIR, int CS>
static hipError_t launch_strided_small_c(const StridedArgs& a) {
  constexpr int T = N1 / lds_epth(N1);
  const int groups = (int)(CS / a.stride);
  const long long blocks = (a.outer + groups - 1) / groups;
  if (a.in_im == nullptr)
    hipLaunchKernelGGL((strided_small_kernel<N1, DIR, true, CS>), dim3((unsigned)blocks), dim3(CS * T), 0, a.stream,
                       a.in_re, a.in_im, a.out_re, a.out_im, a.tw, a.outer, (int)a.stride, groups, a.scale);
  else
    hipLaunchKernelGGL((strided_small_kernel<N1, DIR, false, CS>), dim3((unsigned)blocks), dim3(CS * T), 0, a.stream,
                       a.in_re, a.in_im, a.out_re, a.out_im, a.tw, a.outer, (int)a.stride, groups, a.scale);
  return hipGetLastError();
}

// Column tile of the few-column kernel up to n = 1024: the strided kernel's, narrowed until two
// workgroups fit in a CU's LDS (n = 256 over 3 columns 37.4 -> 30.7 us, 512 55.4 -> 48.8, 1024
// 40.4 -> 31.9; n = 2048 measured 5 % slower and keeps the full tile)
__host__ __device__ constexpr int strided_small_tile(int l) {
  int c = fourstep_tile(l);
  while (c > 1 && (long long)c * (lds_pad(l) + 1) * 8 > kLdsBytes / 2) c /= 2;
  return c;
}

template <int N1, int DIR>
static hipError_t launch_strided_t(const StridedArgs& a) {
  constexpr int C = fourstep_tile(N1), T = N1 / lds_epth(N1);
  if (2 * a.stride <= C) {
    constexpr int CS = strided_small_tile(N1);
    if (N1 <= 1024 && a.stride <= CS) return launch_strided_small_c<N1, DIR, CS>(a);
    return launch_strided_small_c<N1, DIR, C>(a);
  }
  const long long tiles = (a.stride + C - 1) / C;
  const long long blocks = a.outer * tiles;
  if (a.in_im == nullptr)
    hipLaunchKernelGGL((strided_kernel<N1, DIR, true>), dim3((unsigned)blocks), dim3(C * T), 0, a.stream, a.in_re,
                       a.in_im, a.out_re, a.out_im, a.tw, a.stride, (int)tiles, a.scale);
  else
    hipLaunchKernelGGL((strided_kernel<N1, DIR, false>), dim3((unsigned)blocks), dim3(C * T), 0, a.stream, a.in_re,
                       a.in_im, a.out_re, a.out_im, a.tw, a.stride, (int)tiles, a.scale);
  return hipGetLastError();
}

template <int DIR>
static hipError_t launch_strided_dir(int n1, const StridedArgs& a) {
  switch (n1) {
    case 2: return launch_strided_t<2, DIR>(a);
    case 4: return launch_strided_t<4, DIR>(a);
    case 8: return launch_strided_t<8, DIR>(a);
    case 16: return launch_strided_t<16, DIR>(a);
    case 32: return launch_strided_t<32, DIR>(a);
    case 64: return launch_strided_t<64, DIR>(a);
    case 128: return launch_strided_t<128, DIR>(a);
    case 256: return launch_strided_t<256, DIR>(a);
    case 512: return launch_strided_t<512, DIR>(a);
    case 1024: return launch_strided_t<1024, DIR>(a);
    case 2048: return launch_strided_t<2048, DIR>(a);
    case 4096: return launch_strided_t<4096, DIR>(a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_strided(int n1, const StridedArgs& a) {
  return a.dir < 0 ? launch_strided_dir<-1>(n1, a) : launch_strided_dir<1>(n1, a);
}

template <int N1, int N2, int DIR, int TILE_>
static hipError_t launch_fourstep_tiles(const FourStepArgs& a) {
  using C1 = FourStepCfg<N1, TILE_>;
  using C2 = FourStepCfg<N2, TILE_>;
  constexpr int CK = C2::TILE;
  static_assert(N2 % C1::TILE == 0 && N1 % CK == 0, "four-step tiles");
  const unsigned nmask = (unsigned)((long long)N1 * N2 - 1);
  const long long cols = a.batch * (N2 / C1::TILE);
  const bool twl = (1LL << a.lo_bits) + (((long long)N1 * N2) >> a.lo_bits) <= fourstep_twl_cap<N1, TILE_>();
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)cols), dim3(C1::THREADS), 0, a.stream, a.in_re, a.in_im, a.t_re, a.t_im,
                       a.tw1, a.tw_lo, a.tw_hi, (long long)N2, N2 / C1::TILE, a.lo_bits, nmask);
  };
  if (a.in_im == nullptr) {
    if (twl) go(fourstep_col_kernel<N1, DIR, true, CK, TILE_, true>);
    else go(fourstep_col_kernel<N1, DIR, true, CK, TILE_, false>);
  } else {
    if (twl) go(fourstep_col_kernel<N1, DIR, false, CK, TILE_, true>);
    else go(fourstep_col_kernel<N1, DIR, false, CK, TILE_, false>);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long long rows = a.batch * (N1 / CK);
  constexpr bool ROW_TWL = make_shape(N2, C2::E).twoff[make_shape(N2, C2::E).npass] <= fourstep_twl_cap<N2, TILE_>();
  hipLaunchKernelGGL((fourstep_row_kernel<N2, DIR, TILE_, ROW_TWL>), dim3((unsigned)rows), dim3(C2::THREADS), 0,
                     a.stream, a.t_re, a.t_im, a.out_re, a.out_im, a.tw2, N1, a.scale);
  return hipGetLastError();
}

template <int N1, int N2, int DIR>
static hipError_t launch_fourstep_t(const FourStepArgs& a) {
  // a batch whose wide-tile column pass would fill fewer than half the CUs runs narrow tiles
  // (four times the workgroups): 1 x 2^20 35.5 -> 22.2 us, 1 x 2^16 14.0 -> 9.9, 2 x 2^20 36.3 ->
  // 26.1; at 4 x 2^20 (128 wide workgroups) the wide tiles stay faster (40.4 against 44.2)
  if (a.batch * (N2 / FourStepCfg<N1>::TILE) < kNumCUs / 2 && FourStepCfg<N1>::TILE > kFourStepNarrow &&
      FourStepCfg<N2>::TILE > kFourStepNarrow)
    return launch_fourstep_tiles<N1, N2, DIR, kFourStepNarrow>(a);
  return launch_fourstep_tiles<N1, N2, DIR, 0>(a);
}

// n = n1 * n2 (the plan's split: n1 = 2^floor(lg/2) <= n2, or n1 = 2 n2 at 2^15 and 2^17)
template <int DIR>
static hipError_t launch_fourstep_dir(const FourStepArgs& a) {
  const long long key = (long long)a.n1 * 8192 + a.n2;
  switch (key) {
    case 256LL * 8192 + 128: return launch_fourstep_t<256, 128, DIR>(a);
    case 512LL * 8192 + 256: return launch_fourstep_t<512, 256, DIR>(a);
    case 256LL * 8192 + 256: return launch_fourstep_t<256, 256, DIR>(a);
    case 512LL * 8192 + 512: return launch_fourstep_t<512, 512, DIR>(a);
    case 512LL * 8192 + 1024: return launch_fourstep_t<512, 1024, DIR>(a);
    case 1024LL * 8192 + 1024: return launch_fourstep_t<1024, 1024, DIR>(a);
    case 1024LL * 8192 + 2048: return launch_fourstep_t<1024, 2048, DIR>(a);
    case 2048LL * 8192 + 2048: return launch_fourstep_t<2048, 2048, DIR>(a);
    case 2048LL * 8192 + 4096: return launch_fourstep_t<2048, 4096, DIR>(a);
    case 4096LL * 8192 + 4096: return launch_fourstep_t<4096, 4096, DIR>(a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fourstep(const FourStepArgs& a) {
  return a.dir < 0 ? launch_fourstep_dir<-1>(a) : launch_fourstep_dir<1>(a);
}

}  // namespace tfa
