// Two-pass 2-D FFT over the last two axes of a (batch, H, W) array, trnfft/api.py:105-139
// (fft2 -> fftn over dims (-2, -1), which the reference runs as two transposed 1-D passes).
//
// The length-H column transform is split as H = 8 * HR (row r = r1 + HR*j, output q = q2 + 8*q1):
//   Y[q2 + 8 q1] = sum_r1 W_HR^(r1 q1) [ W_H^(r1 q2) sum_j x[r1 + HR j] W_8^(j q2) ]
// Pass 1 (input -> output): one workgroup takes the 8 rows {r1 + HR*j}, transforms each along W
//         (LDS Stockham), then applies the 8-point DFT across those rows and the twiddle
//         W_H^(r1 q2), and writes the 8 results as the consecutive rows 8*r1 + q2: every HBM
//         access is a whole contiguous row.
// Real input: pass 1 pairs rows and writes columns 0..W/2 only; pass 2 transforms those and
//         writes each column w < W/2 a second time as column W-w (2-D Hermitian symmetry), so
//         the half-spectrum is read once and the full spectrum written once.
// Pass 2 (in place on the output): for each group q2, the HR-point transform over r1 of the rows
//         q2 + 8*r1 gives Y[q2 + 8*q1], which lands on row q2 + 8*q1 -- the same row set, so a
//         workgroup (C adjacent columns of one group) reads and then overwrites only its own data.
#include "kernels.h"

namespace tfa {

template <int W>
struct Fft2Row {
  static constexpr int E = lds_epth(W);
  static constexpr int T = W / E;
  static constexpr int THREADS = 8 * T;
  static constexpr int PADW = lds_pad(W);
};

template <int W, int DIR, bool REAL_IN>
__global__ __launch_bounds__(Fft2Row<W>::THREADS) void fft2_pass1_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re, float* out_im,
    const float2* __restrict__ tw_w, const float2* __restrict__ tw_h, int H, int HR) {
  using C = Fft2Row<W>;
  constexpr int E = C::E, T = C::T, PADW = C::PADW;
  static_assert(8 * E >= 16 && (W * 8) % C::THREADS == 0, "layout");
  // the 8 rows as interleaved (re, im) entries, or (W = 4096, 8 rows = 278 KB) one plane at a time
  constexpr bool SPL = 8LL * PADW * 8 > kLdsBytes;
  __shared__ float2 lds[SPL ? 8 * PADW / 2 : 8 * PADW];
  float* lre = reinterpret_cast<float*>(lds);
  const long long g = blockIdx.x;
  const long long b = g / HR;
  const int r1 = (int)(g % HR);
  const int j = threadIdx.x / T;  // which of the block's 8 rows
  const int tid = threadIdx.x % T;
  const size_t img = (size_t)b * H * W;
  const size_t row_in = img + (size_t)(r1 + HR * j) * W;

  float2 v[E];
  {
    const float* pr = in_re + row_in + tid;
    const float* pi = REAL_IN ? nullptr : in_im + row_in + tid;
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = make_float2(ld_stream(pr + T * e), REAL_IN ? 0.0f : ld_stream(pi + T * e));
  }
  // cross-row 8-point DFT: thread t handles columns k = t + THREADS*m, m < W*8/THREADS/8
  constexpr int KPT = W / C::THREADS;  // columns per thread (>= 1 since W >= THREADS/8 * 8)
  float2 zc[SPL ? KPT : 1][8];          // split planes: the columns gathered one plane at a time
  if constexpr (SPL) {
    LdsFft<W, E, DIR, false, true>::run(v, lre + j * PADW, nullptr, tw_w, tid);
#pragma unroll
    for (int plane = 0; plane < 2; ++plane) {
      __syncthreads();  // the previous reads of the buffer are done
#pragma unroll
      for (int e = 0; e < E; ++e) lre[j * PADW + lds_pad(tid + T * e)] = plane ? v[e].y : v[e].x;
      __syncthreads();
#pragma unroll
      for (int m = 0; m < KPT; ++m) {
        const int k = threadIdx.x + C::THREADS * m;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const float f = lre[jj * PADW + lds_pad(k)];
          if (plane) zc[m][jj].y = f;
          else zc[m][jj].x = f;
        }
      }
    }
  } else {
    LdsFft<W, E, DIR, false, false, true>::run(v, reinterpret_cast<float*>(lds + j * PADW), nullptr, tw_w, tid);
#pragma unroll
    for (int e = 0; e < E; ++e) lds[j * PADW + lds_pad(tid + T * e)] = v[e];
    __syncthreads();
  }
  float2 tq[8];
#pragma unroll
  for (int q = 1; q < 8; ++q) tq[q] = tw_h[(r1 * q) & (H - 1)];
#pragma unroll
  for (int m = 0; m < KPT; ++m) {
    const int k = threadIdx.x + C::THREADS * m;
    float2 z[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) z[jj] = SPL ? zc[SPL ? m : 0][jj] : lds[jj * PADW + lds_pad(k)];
    Dft<8, DIR>::run(z);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float2 y = q == 0 ? z[0] : cmul(z[q], tq[q]);
      const size_t o = img + (size_t)(8 * r1 + q) * W + k;
      st_stream(out_re + o, y.x);
      st_stream(out_im + o, y.y);
    }
  }
}

// Real input: the 8 rows form 4 pairs, each pair one complex row transform z = x_2p + i x_2p+1
// (Z = X_2p + i X_2p+1 with both spectra Hermitian), so the row stage costs half the transforms
// and half the LDS; the cross-row stage separates X_2p[k] = (Z[k] + conj Z[W-k]) / 2 and
// X_2p+1[k] = (Z[k] - conj Z[W-k]) / 2i as it reads each column (valid for either sign).
template <int W, int E_ = fft2_pair_epth(W)>
struct Fft2RowPair {
  static constexpr int E = E_;
  static constexpr int T = W / E;
  static constexpr int THREADS = 4 * T;
  static constexpr int PADW = lds_pad(W);
};

template <int W, int DIR, int E_ = fft2_pair_epth(W)>
__global__ __launch_bounds__((Fft2RowPair<W, E_>::THREADS)) void fft2_pass1_real_kernel(
    const float* __restrict__ in, float* out_re, float* out_im, const float2* __restrict__ tw_w,
    const float2* __restrict__ tw_h, int H, int HR) {
  using C = Fft2RowPair<W, E_>;
  constexpr int E = C::E, T = C::T, PADW = C::PADW, THREADS = C::THREADS;
  __shared__ float2 lds[4 * PADW];  // interleaved (re, im)
  const long long g = blockIdx.x;
  const long long b = g / HR;
  const int r1 = (int)(g % HR);
  const int p = threadIdx.x / T;  // pair: rows r1 + HR*(2p) and r1 + HR*(2p+1)
  const int tid = threadIdx.x % T;
  const size_t img = (size_t)b * H * W;
  const float* pa = in + img + (size_t)(r1 + HR * (2 * p)) * W + tid;
  const float* pb = pa + (size_t)HR * W;

  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = make_float2(ld_stream(pa + T * e), ld_stream(pb + T * e));
  LdsFft<W, E, DIR, (T <= 64), false, true>::run(v, reinterpret_cast<float*>(lds + p * PADW), nullptr, tw_w, tid);
#pragma unroll
  for (int e = 0; e < E; ++e) lds[p * PADW + lds_pad(tid + T * e)] = v[e];
  __syncthreads();
  float2 tq[8];
#pragma unroll
  for (int q = 1; q < 8; ++q) tq[q] = tw_h[(r1 * q) & (H - 1)];
  // columns 0..W/2 only: pass 2 completes the rest from the 2-D Hermitian symmetry
  for (int k = threadIdx.x; k <= W / 2; k += THREADS) {
    const int ik = lds_pad(k), ir = lds_pad((W - k) & (W - 1));
    float2 z[8];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const float2 za = lds[pp * PADW + ik], zc = lds[pp * PADW + ir];
      const float ar = za.x, ai = za.y;
      const float cr = zc.x, ci = -zc.y;  // conj Z[W-k]
      z[2 * pp] = make_float2(0.5f * (ar + cr), 0.5f * (ai + ci));
      z[2 * pp + 1] = make_float2(0.5f * (ai - ci), -0.5f * (ar - cr));
    }
    Dft<8, DIR>::run(z);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float2 y = q == 0 ? z[0] : cmul(z[q], tq[q]);
      const size_t o = img + (size_t)(8 * r1 + q) * W + k;
      st_stream(out_re + o, y.x);
      st_stream(out_im + o, y.y);
    }
  }
}

// Pass 2 tile width: columns per workgroup within the LDS and 1024-thread limits (E from
// fft2_col_epth: 8 elements per thread, e.g. HR = 256 -> 32 columns of 32 threads, measured
// 15 % faster than 64 columns of 16 threads).
__host__ __device__ constexpr int fft2_tile(int hr) {
  int c = 64;
  while (c > 1 && ((long long)c * (lds_pad(hr) + 1) * 8 > kLdsBytes || c * (hr / fft2_col_epth(hr)) > 1024)) c /= 2;
  return c;
}

// HALF (real input): pass 1 wrote only columns 0..W/2; each transformed column w in 1..W/2-1 is
// also written, conjugated and row-reflected, as column W-w (X[h][w] = conj X[-h][-w] for a real
// image).  Columns above W/2 are never read, so these writes race with nothing.
template <int HR, int DIR, bool HALF = false, int C = fft2_tile(HR), int E_ = fft2_col_epth(HR)>
__global__ __launch_bounds__(C * (HR / E_)) void fft2_pass2_kernel(
    float* re, float* im, const float2* __restrict__ tw, int W, int tiles_per_group, float scale) {
  constexpr int E = E_, T = HR / E;
  constexpr int PADN = lds_pad(HR) + 1;
  __shared__ float2 lds[C * PADN];  // interleaved (re, im) exchange
  const int c = threadIdx.x % C;
  const int t = threadIdx.x / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long grp = tile / tiles_per_group;  // (image, q2)
  const long long b = grp / 8;
  const int q2 = (int)(grp % 8);
  const int col = (int)(tile % tiles_per_group) * C + c;
  const bool valid = col < (HALF ? W / 2 + 1 : W);
  // element r1 (input) and q1 (output) of column col in group q2 both live at row q2 + 8*index
  const size_t base = (size_t)b * (8 * HR) * W + (size_t)q2 * W + col;
  const size_t step = (size_t)8 * W;
  // a column past the last reads the tile's last column (unconditional loads: under `valid ?`
  // the compiler waited for each load before issuing the next); its results are not stored
  const int ncol = HALF ? W / 2 + 1 : W;
  const size_t lbase = valid ? base : base - (size_t)(col - (ncol - 1));

  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = lbase + (size_t)(t + T * e) * step;
    v[e] = make_float2(ld_stream(re + i) * scale, ld_stream(im + i) * scale);
  }
  // every value this workgroup loads is consumed by the transform (whose first exchange is a
  // workgroup barrier) before any thread stores; no other workgroup touches these elements
  LdsFft<HR, E, DIR, false, false, true>::run(v, reinterpret_cast<float*>(lds + c * PADN), nullptr, tw, t);
  if (!valid) return;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t o = base + (size_t)(t + T * e) * step;
    st_stream(re + o, v[e].x);
    st_stream(im + o, v[e].y);
  }
  if constexpr (HALF) {
    if (col >= 1 && col < W / 2) {
      constexpr int H = 8 * HR;
      const size_t mb = (size_t)b * H * W + (size_t)(W - col);
      // the mirror of an aligned column tile [w0, w0 + C) is [W - w0 - C + 1, W - w0]: one
      // column off the line grid, so plain stores (L2 merges the neighbouring tile's halves)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int h = q2 + 8 * (t + T * e);
        const size_t o = mb + (size_t)((H - h) & (H - 1)) * W;
        re[o] = v[e].x;
        im[o] = -v[e].y;
      }
    }
  }
}

// Real input, pass 2 with whole-line mirror stores.  The mirror of the column tile [C*T, C*T + C)
// is [W - C*T - C + 1, W - C*T]: one column off the line grid.  The aligned run
// [W - C*T - C, W - C*T) instead holds the mirrors of columns C*T + 1 .. C*T + C, where the last
// column is the first column of tile T + 1.  So a workgroup takes a run of adjacent tiles of one
// group in descending order.  Each tile's lane-0 threads keep their column's mirrored values
// (the "carry", in LDS slots that only the owning thread touches) for the next tile, whose mirror
// stores then cover whole aligned lines.  The first tile of a run has no carry: its lane 0 stores
// its own mirrored column instead (the next tile's carry store repeats it), and the first column
// of its line comes from the run above, which stores its last carry after its loop; those
// partial lines take plain stores.
// Column W/2 (lane 0 of the top tile, W/2 being a multiple of C) is its own mirror and is read by
// the workgroup of its own group, so it is only stored in place, never as a carry (a carry would
// be written by the workgroup of the mirrored group, which may run first): the line starting at
// W/2 is split like a run's first line.
// The tile loop is software-pipelined: the next tile's loads are issued before this tile's
// stores, and the twiddle table is staged in LDS once, so the transform issues no global loads
// (gfx9 counts loads and stores in one in-order counter: waiting for a load issued after a store
// also waits for the store).  The first and last tiles are peeled, so every path into a tile
// holds the same outstanding loads and stores and the compiler's waits cover the loads only.
template <int HR, int DIR, int C = fft2_tile(HR), int E_ = fft2_col_epth(HR)>
__global__ __launch_bounds__(C * (HR / E_)) void fft2_pass2_half_kernel(
    float* re, float* im, const float2* __restrict__ tw, int W, int tiles_per_group, int runs, float scale) {
  constexpr int E = E_, T = HR / E;
  constexpr int PADN = lds_pad(HR) + 1;
  constexpr int H = 8 * HR;
  constexpr int NTW = make_shape(HR, E).twoff[make_shape(HR, E).npass];  // twiddle entries
  __shared__ float2 lds[C * PADN];  // interleaved (re, im) exchange
  __shared__ float2 carry[2 * T * E];  // lane-0 threads' mirrored column, slot (tile & 1, t, e)
  __shared__ __attribute__((aligned(16))) float2 twl[NTW > 0 ? NTW : 2];
  const int c = threadIdx.x % C;
  const int t = threadIdx.x / C;
  const unsigned grp = blockIdx.x / (unsigned)runs;  // (image, q2)
  const int run = (int)(blockIdx.x - grp * (unsigned)runs);
  const unsigned q2 = grp % 8u;
  // run r takes tiles [r * TPG / runs, (r + 1) * TPG / runs) (at least two: runs <= TPG / 2)
  const int lo = run * tiles_per_group / runs;
  const int hi = (run + 1) * tiles_per_group / runs - 1;
  const int half = W / 2;
  const int top = half / C;  // tile of column W/2 (>= 2)
  // the image's planes (workgroup-uniform bases) and 32-bit byte offsets within the image
  // (H * W * 4 < 2^32)
  const size_t img = (size_t)(grp / 8u) * H * W;
  char* const bre = reinterpret_cast<char*>(re + img);
  char* const bim = reinterpret_cast<char*>(im + img);
  const unsigned Wb = 4u * (unsigned)W;
  const unsigned estep = 8u * T * Wb;  // element e of a thread is 8 T e rows further
  // row q2 + 8t, and the mirror rows (H - q2 - 8t - 8Te) mod H: only e = 0 can wrap (to row 0)
  const unsigned row_t0 = (q2 + 8u * (unsigned)t) * Wb;
  const unsigned mrow_t = (unsigned)H - q2 - 8u * (unsigned)t;
  const unsigned mrow0_0 = (mrow_t & (unsigned)(H - 1)) * Wb;
  const unsigned mrow1_0 = mrow_t * Wb;
  // lanes past column W/2 (top tile only) load, transform and store a copy of column W/2: the
  // columns transform independently, so they store the same values as lane 0
  auto load = [&](int tile, float2 (&x)[E]) {
    const int col = tile * C + c;
    const unsigned cb = 4u * (unsigned)(col <= half ? col : half);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const unsigned o = row_t0 + e * estep + cb;
      x[e] = make_float2(__builtin_nontemporal_load(reinterpret_cast<const float*>(bre + o)),
                         __builtin_nontemporal_load(reinterpret_cast<const float*>(bim + o)));
    }
  };
  float2 nx[E];
  load(hi, nx);
  for (int i = threadIdx.x; i < NTW; i += C * T) twl[i] = tw[i];
  __syncthreads();
  // one tile: transform the loaded values, request the next tile's (PF), store this one's
  auto step = [&](int tile, bool pf) {
    // recomputed per tile (the empty asm hides their loop invariance): the compiler would
    // otherwise keep the eight elements' row and mirror offsets in registers across the loop
    // (over 100 VGPRs against ~76)
    unsigned row_t = row_t0, mrow0 = mrow0_0, mrow1 = mrow1_0;
    int cc = c;
    asm volatile("" : "+v"(row_t), "+v"(mrow0), "+v"(mrow1), "+v"(cc));
    float2 v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = make_float2(nx[e].x * scale, nx[e].y * scale);
    // the previous tile's transform ended with a barrier after its last LDS reads
    LdsFft<HR, E, DIR, false, false, true>::run(v, reinterpret_cast<float*>(lds + c * PADN), nullptr, twl, t);
    // the next tile's loads go out once the transform's temporaries are dead (register pressure)
    __builtin_amdgcn_sched_barrier(0);
    if (pf) load(tile - 1, nx);
    __builtin_amdgcn_sched_barrier(0);
    const int col = tile * C + cc;
    const unsigned cb = 4u * (unsigned)(col <= half ? col : half);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const unsigned o = row_t + e * estep + cb;
      st_stream(reinterpret_cast<float*>(bre + o), v[e].x);
      st_stream(reinterpret_cast<float*>(bim + o), v[e].y);
    }
    // mirror: lane c >= 1 stores column W - col, lane 0 the carry (mirror of column col + C) as
    // the line's first column W - col - C, or without a carry its own mirror W - col.  The top
    // tile (column W/2 only: no mirror) repeats its in-place stores instead, so that every tile
    // issues the same stores; its carry is never used.
    // The carry slots alternate by tile parity: lane 0 writes its new carry first and then reads
    // the previous tile's into v (conjugated, as the stores conjugate v), so both never occupy
    // registers at once.
    const bool at_top = tile == top;
    const bool has_carry = tile < hi && tile + 1 < top;
    const bool use_carry = has_carry && cc == 0;
    if (cc == 0) {
#pragma unroll
      for (int e = 0; e < E; ++e) carry[(tile & 1) * T * E + t * E + e] = make_float2(v[e].x, -v[e].y);
      if (use_carry) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float2 y = carry[((tile + 1) & 1) * T * E + t * E + e];
          v[e] = make_float2(y.x, -y.y);
        }
      }
    }
    const unsigned mc = 4u * (unsigned)(W - col - (use_carry ? C : 0));
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const unsigned o = at_top ? row_t + e * estep + cb : (e == 0 ? mrow0 : mrow1 - e * estep) + mc;
      float* pr = reinterpret_cast<float*>(bre + o);
      float* pi = reinterpret_cast<float*>(bim + o);
      const float yi = at_top ? v[e].y : -v[e].y;
      if (has_carry) {  // whole line with lane 0's carry
        st_stream(pr, v[e].x);
        st_stream(pi, yi);
      } else {  // the run's first tile: the line's first column comes from the run above
        *pr = v[e].x;
        *pi = yi;
      }
    }
  };
  step(hi, true);
  for (int tile = hi - 1; tile > lo; --tile) step(tile, true);
  step(lo, false);
  // the last tile's carry (mirror of column C*lo) opens the first mirror line of the run below
  if (c == 0 && lo >= 1 && lo < top) {
    const unsigned mc = 4u * (unsigned)(W - lo * C);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float2 y = carry[(lo & 1) * T * E + t * E + e];
      const unsigned o = (e == 0 ? mrow0_0 : mrow1_0 - e * estep) + mc;
      *reinterpret_cast<float*>(bre + o) = y.x;
      *reinterpret_cast<float*>(bim + o) = y.y;
    }
  }
}

// Runs per group of the whole-line pass 2 (0: the one-tile-per-workgroup kernel), from an in-run
// sweep on MI355X (real input, whole fft2, us; old = one tile per workgroup): one workgroup per
// CU in all (the kernel holds ~76 VGPRs: one 1024-thread workgroup per CU) was fastest at every
// shape: 32 x 2048^2 582 (2 runs 599, 4 runs 632; old 622), 16 x 1024^2 73.3 (old 82.2), 64 x 512^2
// 69.0 (old 80.6), 8 x 2048 x 1024 77.9 (old 83.9).  When that would need runs of fewer than two
// tiles the old kernel stays (1 x 2048^2: 29.9 against 36.6 with 16 runs).  Tiles must cover at
// least one 128-byte line, with W/2 a multiple of the tile and at least two tiles below it.
static int fft2_half_runs(long long groups, int tiles, int c, int w) {
  if (c < 32 || (w / 2) % c != 0 || w / 2 < 2 * c) return 0;
  const long long runs = (kNumCUs + groups - 1) / groups;
  return runs > tiles / 2 ? 0 : (int)runs;
}

template <int W, int DIR>
static hipError_t launch_pass1_w(const Fft2Args& a) {
  const long long blocks = a.batch * (a.h / 8);
  if (a.in_im == nullptr)  // real input: paired rows (measured 504 -> 299 us at 32 x 2048^2)
    hipLaunchKernelGGL((fft2_pass1_real_kernel<W, DIR>), dim3((unsigned)blocks), dim3(Fft2RowPair<W>::THREADS), 0,
                       a.stream, a.in_re, a.out_re, a.out_im, a.tw_w_pair, a.tw_h, a.h, a.h / 8);
  else
    hipLaunchKernelGGL((fft2_pass1_kernel<W, DIR, false>), dim3((unsigned)blocks), dim3(Fft2Row<W>::THREADS), 0,
                       a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw_w, a.tw_h, a.h, a.h / 8);
  return hipGetLastError();
}

template <int HR, int DIR>
static hipError_t launch_pass2_h(const Fft2Args& a) {
  constexpr int C = fft2_tile(HR), T = HR / fft2_col_epth(HR);
  const bool half = a.in_im == nullptr;  // real input: pass 1 wrote columns 0..W/2
  const int tiles = (int)(((half ? a.w / 2 + 1 : a.w) + C - 1) / C);
  const long long blocks = a.batch * 8 * (long long)tiles;
  const int runs = half ? fft2_half_runs(a.batch * 8, tiles, C, (int)a.w) : 0;
  if (runs > 0)
    hipLaunchKernelGGL((fft2_pass2_half_kernel<HR, DIR>), dim3((unsigned)(a.batch * 8 * runs)), dim3(C * T), 0,
                       a.stream, a.out_re, a.out_im, a.tw_hr, (int)a.w, tiles, runs, a.scale);
  else if (half)
    hipLaunchKernelGGL((fft2_pass2_kernel<HR, DIR, true>), dim3((unsigned)blocks), dim3(C * T), 0, a.stream,
                       a.out_re, a.out_im, a.tw_hr, (int)a.w, tiles, a.scale);
  else
    hipLaunchKernelGGL((fft2_pass2_kernel<HR, DIR, false>), dim3((unsigned)blocks), dim3(C * T), 0, a.stream,
                       a.out_re, a.out_im, a.tw_hr, (int)a.w, tiles, a.scale);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Single-pass small images (h*w <= 16384): one HBM read and one HBM write per element.  The
// workgroup's IMG images are staged row-major into LDS (row r of image i at (i*H + r)*RW, entry c
// at lds_pad(c)); every row is transformed with its own LDS row as the exchange area, written
// back transposed (column k at (i*W + k)*CH, entry r at lds_pad(r)); every column is transformed
// in place the same way; the store phase reads the columns back in row order.
// ---------------------------------------------------------------------------------------------
template <int H, int W>
struct Fft2SmallCfg {
  static constexpr int IMG = fft2_small_img(H, W);
  static constexpr int E = fft2_small_epth(H, W);
  static constexpr int TW = W / E, TH = H / E;   // threads per row / per column
  static constexpr int THREADS = 1024;
  static constexpr int RW = lds_pad(W) + 1, CH = lds_pad(H) + 1;  // odd pitches
  static constexpr int PER = H * RW > W * CH ? H * RW : W * CH;    // float2 entries per image
  static constexpr int P = H * W;
  static_assert(IMG * H * TW == THREADS && IMG * W * TH == THREADS, "one row / column per thread group");
  static_assert((long long)IMG * PER * 8 <= kLdsBytes, "small-image tile exceeds LDS");
};

template <int H, int W, int DIR, bool REAL_IN, bool TAIL>
__global__ __launch_bounds__(1024) void fft2_small_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw_w, const float2* __restrict__ tw_h,
    long long first, long long batch, float scale) {
  using C = Fft2SmallCfg<H, W>;
  constexpr int E = C::E, TW = C::TW, TH = C::TH, RW = C::RW, CH = C::CH, P = C::P, IMG = C::IMG;
  __shared__ float2 lds[IMG * C::PER];
  const long long i0 = first + (long long)blockIdx.x * IMG;  // first image of the tile
  const int count = TAIL ? (int)((batch - i0 < IMG ? batch - i0 : IMG) * P) : IMG * P;
  const size_t g0 = (size_t)i0 * P;
  const float sc = DIR < 0 ? 1.0f : scale;  // inverse: 1/(h*w) on the input (exact, powers of two)
  // E loads per thread, all issued before the first LDS write (a ragged tail rereads its last
  // element)
  static_assert(IMG * P == 1024 * E, "the tile's floats per plane are E steps of the workgroup");
  float xr[E], xi[E];
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int i = (int)threadIdx.x + 1024 * u;
    const int ic = TAIL && i >= count ? count - 1 : i;
    xr[u] = ld_stream(in_re + g0 + ic);
    xi[u] = REAL_IN ? 0.0f : ld_stream(in_im + g0 + ic);
  }
  __builtin_amdgcn_sched_barrier(0);  // (else the scheduler pairs each load with its write)
#pragma unroll
  for (int u = 0; u < E; ++u) {
    const int i = (int)threadIdx.x + 1024 * u;
    if (!TAIL || i < count) {
      const int img = i / P, r = (i % P) / W, c = i % W;
      lds[(img * H + r) * RW + lds_pad(c)] = make_float2(xr[u] * sc, xi[u] * sc);
    }
  }
  __syncthreads();
  float2 v[E];
  {  // rows (images past a ragged tail hold stale LDS data: transformed, never stored)
    const int row = threadIdx.x / TW, tid = threadIdx.x % TW;  // row = img*H + r
    float2* base = lds + row * RW;
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = base[lds_pad(tid + TW * e)];
    __syncthreads();  // the row area becomes the transform's exchange area
    LdsFft<W, E, DIR, (TW <= 64), false, true>::run(v, reinterpret_cast<float*>(base), nullptr, tw_w, tid);
    __syncthreads();
    const int img = row / H, r = row % H;
#pragma unroll
    for (int e = 0; e < E; ++e) lds[(img * W + tid + TW * e) * CH + lds_pad(r)] = v[e];
    __syncthreads();
  }
  {  // columns
    const int col = threadIdx.x / TH, tid = threadIdx.x % TH;  // col = img*W + k
    float2* base = lds + col * CH;
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = base[lds_pad(tid + TH * e)];
    __syncthreads();
    LdsFft<H, E, DIR, (TH <= 64), false, true>::run(v, reinterpret_cast<float*>(base), nullptr, tw_h, tid);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) base[lds_pad(tid + TH * e)] = v[e];
    __syncthreads();
  }
  for (int i = threadIdx.x; i < count; i += 1024) {
    const int img = i / P, q = (i % P) / W, k = i % W;
    const float2 y = lds[(img * W + k) * CH + lds_pad(q)];
    st_stream(out_re + g0 + i, y.x);
    st_stream(out_im + g0 + i, y.y);
  }
}

template <int H, int W, int DIR>
static hipError_t launch_fft2_small_hw(const Fft2Args& a) {
  if constexpr (fft2_small_ok(H, W)) {
    using C = Fft2SmallCfg<H, W>;
    const long long blocks = (a.batch + C::IMG - 1) / C::IMG;
    const bool real_in = a.in_im == nullptr;
    if (blocks * C::IMG == a.batch) {
      if (real_in)
        hipLaunchKernelGGL((fft2_small_kernel<H, W, DIR, true, false>), dim3((unsigned)blocks), dim3(1024), 0,
                           a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw_sw, a.tw_sh, 0LL, a.batch, a.scale);
      else
        hipLaunchKernelGGL((fft2_small_kernel<H, W, DIR, false, false>), dim3((unsigned)blocks), dim3(1024), 0,
                           a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw_sw, a.tw_sh, 0LL, a.batch, a.scale);
    } else {  // ragged batch: one launch of the guarded variant
      if (real_in)
        hipLaunchKernelGGL((fft2_small_kernel<H, W, DIR, true, true>), dim3((unsigned)blocks), dim3(1024), 0,
                           a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw_sw, a.tw_sh, 0LL, a.batch, a.scale);
      else
        hipLaunchKernelGGL((fft2_small_kernel<H, W, DIR, false, true>), dim3((unsigned)blocks), dim3(1024), 0,
                           a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw_sw, a.tw_sh, 0LL, a.batch, a.scale);
    }
    return hipGetLastError();
  } else {
    return hipErrorInvalidValue;
  }
}

template <int H, int DIR>
static hipError_t launch_fft2_small_h(const Fft2Args& a) {
  switch (a.w) {
    case 4: return launch_fft2_small_hw<H, 4, DIR>(a);
    case 8: return launch_fft2_small_hw<H, 8, DIR>(a);
    case 16: return launch_fft2_small_hw<H, 16, DIR>(a);
    case 32: return launch_fft2_small_hw<H, 32, DIR>(a);
    case 64: return launch_fft2_small_hw<H, 64, DIR>(a);
    case 128: return launch_fft2_small_hw<H, 128, DIR>(a);
    case 256: return launch_fft2_small_hw<H, 256, DIR>(a);
    case 512: return launch_fft2_small_hw<H, 512, DIR>(a);
    case 1024: return launch_fft2_small_hw<H, 1024, DIR>(a);
    default: return hipErrorInvalidValue;
  }
}

template <int DIR>
static hipError_t launch_fft2_small(const Fft2Args& a) {
  switch (a.h) {
    case 4: return launch_fft2_small_h<4, DIR>(a);
    case 8: return launch_fft2_small_h<8, DIR>(a);
    case 16: return launch_fft2_small_h<16, DIR>(a);
    case 32: return launch_fft2_small_h<32, DIR>(a);
    case 64: return launch_fft2_small_h<64, DIR>(a);
    case 128: return launch_fft2_small_h<128, DIR>(a);
    case 256: return launch_fft2_small_h<256, DIR>(a);
    case 512: return launch_fft2_small_h<512, DIR>(a);
    case 1024: return launch_fft2_small_h<1024, DIR>(a);
    default: return hipErrorInvalidValue;
  }
}

template <int DIR>
static hipError_t launch_fft2_dir(const Fft2Args& a) {
  if (fft2_small_ok(a.h, a.w)) return launch_fft2_small<DIR>(a);
  hipError_t e;
  switch (a.w) {  // 8 rows x W/E threads must fit one 1024-thread workgroup (W = 4096: E = 32, split planes)
    case 16: e = launch_pass1_w<16, DIR>(a); break;
    case 32: e = launch_pass1_w<32, DIR>(a); break;
    case 64: e = launch_pass1_w<64, DIR>(a); break;
    case 128: e = launch_pass1_w<128, DIR>(a); break;
    case 256: e = launch_pass1_w<256, DIR>(a); break;
    case 512: e = launch_pass1_w<512, DIR>(a); break;
    case 1024: e = launch_pass1_w<1024, DIR>(a); break;
    case 2048: e = launch_pass1_w<2048, DIR>(a); break;
    case 4096: e = launch_pass1_w<4096, DIR>(a); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  switch (a.h / 8) {
    case 2: return launch_pass2_h<2, DIR>(a);
    case 4: return launch_pass2_h<4, DIR>(a);
    case 8: return launch_pass2_h<8, DIR>(a);
    case 16: return launch_pass2_h<16, DIR>(a);
    case 32: return launch_pass2_h<32, DIR>(a);
    case 64: return launch_pass2_h<64, DIR>(a);
    case 128: return launch_pass2_h<128, DIR>(a);
    case 256: return launch_pass2_h<256, DIR>(a);
    case 512: return launch_pass2_h<512, DIR>(a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fft2(const Fft2Args& a) { return a.dir < 0 ? launch_fft2_dir<-1>(a) : launch_fft2_dir<1>(a); }

}  // namespace tfa
