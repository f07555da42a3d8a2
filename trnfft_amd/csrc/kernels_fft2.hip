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
  __shared__ float2 lds[8 * PADW];  // interleaved (re, im)
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
  LdsFft<W, E, DIR, false, false, true>::run(v, reinterpret_cast<float*>(lds + j * PADW), nullptr, tw_w, tid);
#pragma unroll
  for (int e = 0; e < E; ++e) lds[j * PADW + lds_pad(tid + T * e)] = v[e];
  __syncthreads();
  // cross-row 8-point DFT: thread t handles columns k = t + THREADS*m, m < W*8/THREADS/8
  constexpr int KPT = W / C::THREADS;  // columns per thread (>= 1 since W >= THREADS/8 * 8)
  float2 tq[8];
#pragma unroll
  for (int q = 1; q < 8; ++q) tq[q] = tw_h[(r1 * q) & (H - 1)];
#pragma unroll
  for (int m = 0; m < KPT; ++m) {
    const int k = threadIdx.x + C::THREADS * m;
    float2 z[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) z[jj] = lds[jj * PADW + lds_pad(k)];
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

  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = base + (size_t)(t + T * e) * step;
    v[e] = valid ? make_float2(ld_stream(re + i) * scale, ld_stream(im + i) * scale) : make_float2(0.0f, 0.0f);
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
  if (half)
    hipLaunchKernelGGL((fft2_pass2_kernel<HR, DIR, true>), dim3((unsigned)blocks), dim3(C * T), 0, a.stream,
                       a.out_re, a.out_im, a.tw_hr, (int)a.w, tiles, a.scale);
  else
    hipLaunchKernelGGL((fft2_pass2_kernel<HR, DIR, false>), dim3((unsigned)blocks), dim3(C * T), 0, a.stream,
                       a.out_re, a.out_im, a.tw_hr, (int)a.w, tiles, a.scale);
  return hipGetLastError();
}

template <int DIR>
static hipError_t launch_fft2_dir(const Fft2Args& a) {
  hipError_t e;
  switch (a.w) {  // 8 rows x W/E threads must fit one 1024-thread workgroup: W <= 2048
    case 16: e = launch_pass1_w<16, DIR>(a); break;
    case 32: e = launch_pass1_w<32, DIR>(a); break;
    case 64: e = launch_pass1_w<64, DIR>(a); break;
    case 128: e = launch_pass1_w<128, DIR>(a); break;
    case 256: e = launch_pass1_w<256, DIR>(a); break;
    case 512: e = launch_pass1_w<512, DIR>(a); break;
    case 1024: e = launch_pass1_w<1024, DIR>(a); break;
    case 2048: e = launch_pass1_w<2048, DIR>(a); break;
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
