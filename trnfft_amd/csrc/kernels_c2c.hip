// Batched power-of-two complex-to-complex FFT kernels.
//
//  * c2c_lds_kernel: one launch per batch; each transform of length N <= 16384 stays in
//    registers + LDS for all its passes (replaces the reference's per-stage launches,
//    trnfft/fft_core.py:53-117 on CPU and :1063-1238 on the NKI path).
//  * strided_kernel: transform along a non-contiguous axis (element stride S), C adjacent
//    columns per workgroup; replaces the transpose copies of trnfft/api.py:496-516 for fftn/fft2
//    and is the column pass of the four-step path.
//  * four-step (strided_kernel with twiddle + fourstep_row_kernel): N = N1*N2 > 16384 in two HBM
//    passes (column FFTs with the W_N^{n2*k1} twiddle fused into their store, then row FFTs whose
//    output is transposed through LDS so the strided store stays coalesced).  This is the
//    single-GPU form of the reference's row-column decomposition, trnfft/nki/multicore.py:151-219.
#include "kernels.h"

namespace tfa {

// ---------------------------------------------------------------------------------------------
// LDS-resident batched transform
// ---------------------------------------------------------------------------------------------
// TAIL = false: every transform slot of the grid is inside the batch (no guards at all; the
// guard-free instruction stream measured fastest).  TAIL = true: one workgroup for the ragged
// remainder, slots past the batch end neither load nor store.
template <int N, int DIR, bool REAL_IN, bool TAIL, int E_ = c2c_epth(N), int THR = c2c_threads(N)>
__global__ __launch_bounds__((C2cThreads<N, E_, THR>::THREADS)) void c2c_lds_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re,
    float* out_im, const float2* __restrict__ tw, long long first, long long batch, float scale) {
  using C = C2cThreads<N, E_, THR>;
  constexpr int E = C::E, T = C::T;
  __shared__ float lre[C::XF * C::PADN];
  __shared__ float lim[C::XF * C::PADN];
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
  LdsFft<N, E, DIR, (T <= 64)>::run(v, lre + xf * C::PADN, lim + xf * C::PADN, tw, tid);
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

template <int N, int DIR, bool REAL_IN>
static hipError_t launch_c2c_lds_t(const C2cArgs& a) {
  using C = C2cThreads<N>;
  const long long full = a.batch / C::XF;
  if (full > 0)
    hipLaunchKernelGGL((c2c_lds_kernel<N, DIR, REAL_IN, false>), dim3((unsigned)full), dim3(C::THREADS), 0,
                       a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw, 0LL, a.batch, a.scale);
  if (full * C::XF < a.batch)
    hipLaunchKernelGGL((c2c_lds_kernel<N, DIR, REAL_IN, true>), dim3(1), dim3(C::THREADS), 0, a.stream, a.in_re,
                       a.in_im, a.out_re, a.out_im, a.tw, full * C::XF, a.batch, a.scale);
  return hipGetLastError();
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
// Four-step: x viewed as (N1 rows) x (N2 columns), n = N2*n1 + n2, k = k1 + N1*k2.
// ---------------------------------------------------------------------------------------------
// Strided-axis transform: x viewed as (outer, N1, S) row-major; transform along the N1 axis
// (element stride S) for every (outer, column) pair.  One workgroup = C adjacent columns of one
// outer block, so each load/store instruction covers C consecutive floats.  With TWIDDLE the
// result k1 of column c is multiplied by W_Ntot^(c*k1) (the four-step column pass, with S = N2).
template <int N1, int DIR, bool REAL_IN, bool TWIDDLE, int C = fourstep_tile(N1)>
__global__ __launch_bounds__(C * (N1 / lds_epth(N1))) void strided_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re, float* out_im,
    const float2* __restrict__ tw, const float2* __restrict__ tw_lo, const float2* __restrict__ tw_hi,
    long long stride, int tiles_per_block, int lo_bits, unsigned nmask, float scale) {
  constexpr int E = lds_epth(N1), T = N1 / E;
  constexpr int PADN = lds_pad(N1) + 1;
  __shared__ float lre[C * PADN];
  __shared__ float lim[C * PADN];
  const int c = threadIdx.x % C;  // column within tile (fast across lanes: coalesced)
  const int t = threadIdx.x / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_block;
  const long long col = (tile % tiles_per_block) * C + c;
  const bool valid = col < stride;
  const size_t base = (size_t)b * N1 * stride + col;

  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = base + (size_t)(t + T * e) * stride;
    v[e] = valid ? make_float2(ld_stream(in_re + i), REAL_IN ? 0.0f : ld_stream(in_im + i)) : make_float2(0.0f, 0.0f);
  }
  LdsFft<N1, E, DIR, false>::run(v, lre + c * PADN, lim + c * PADN, tw, t);
  if (!valid) return;
  const unsigned lomask = (1u << lo_bits) - 1;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k1 = t + T * e;
    float2 y = v[e];
    if constexpr (TWIDDLE) {
      const unsigned m = ((unsigned)col * (unsigned)k1) & nmask;
      y = cmul(y, cmul(tw_lo[m & lomask], tw_hi[m >> lo_bits]));
    } else {
      y = cscale(y, scale);
    }
    const size_t i = base + (size_t)k1 * stride;
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

// Row pass: FFT over n2 of each row k1 of tmp (contiguous), output X[k1 + N1*k2] for C
// adjacent rows, transposed through LDS so each store covers C consecutive k1.
template <int N2, int DIR, int C = fourstep_tile(N2)>
__global__ __launch_bounds__(C * (N2 / lds_epth(N2))) void fourstep_row_kernel(
    const float* __restrict__ t_re, const float* __restrict__ t_im, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, int n1_len, long long batch,
    float scale) {
  constexpr int E = lds_epth(N2), T = N2 / E;
  constexpr int PADN = lds_pad(N2) + 1;
  constexpr int THREADS = C * T;
  __shared__ float lre[C * PADN];
  __shared__ float lim[C * PADN];
  const int t = threadIdx.x % T;  // position in row (fast across lanes: coalesced loads)
  const int r = threadIdx.x / T;
  const int tiles_per_b = n1_len / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_b;
  const int k1_0 = (int)(tile % tiles_per_b) * C;
  const size_t N = (size_t)n1_len * N2;
  const size_t row_base = (size_t)b * N + (size_t)(k1_0 + r) * N2;

  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = row_base + t + T * e;
    v[e] = make_float2(t_re[i], t_im[i]);
  }
  LdsFft<N2, E, DIR, false>::run(v, lre + r * PADN, lim + r * PADN, tw, t);
  // transpose: element (row r, k2) -> LDS[r*PADN + k2], read back with the row index fast
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int idx = r * PADN + lds_pad(t + T * e);
    lre[idx] = v[e].x;
    lim[idx] = v[e].y;
  }
  __syncthreads();
  const int rr = threadIdx.x % C;
  const int q = threadIdx.x / C;
  constexpr int QN = THREADS / C;  // == T
  const size_t obase = (size_t)b * N + k1_0 + rr;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k2 = q + QN * e;
    const int idx = rr * PADN + lds_pad(k2);
    const size_t o = obase + (size_t)k2 * n1_len;
    out_re[o] = lre[idx] * scale;
    out_im[o] = lim[idx] * scale;
  }
  (void)batch;
}

template <int N1, int DIR, bool TWIDDLE>
static hipError_t launch_strided_t(const StridedArgs& a) {
  constexpr int C = fourstep_tile(N1), T = N1 / lds_epth(N1);
  const long long tiles = (a.stride + C - 1) / C;
  const long long blocks = a.outer * tiles;
  if (a.in_im == nullptr)
    hipLaunchKernelGGL((strided_kernel<N1, DIR, true, TWIDDLE>), dim3((unsigned)blocks), dim3(C * T), 0,
                       a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw, a.tw_lo, a.tw_hi, a.stride,
                       (int)tiles, a.lo_bits, a.nmask, a.scale);
  else
    hipLaunchKernelGGL((strided_kernel<N1, DIR, false, TWIDDLE>), dim3((unsigned)blocks), dim3(C * T), 0,
                       a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw, a.tw_lo, a.tw_hi, a.stride,
                       (int)tiles, a.lo_bits, a.nmask, a.scale);
  return hipGetLastError();
}

template <int DIR, bool TWIDDLE>
static hipError_t launch_strided_dir(int n1, const StridedArgs& a) {
  switch (n1) {
    case 2: return launch_strided_t<2, DIR, TWIDDLE>(a);
    case 4: return launch_strided_t<4, DIR, TWIDDLE>(a);
    case 8: return launch_strided_t<8, DIR, TWIDDLE>(a);
    case 16: return launch_strided_t<16, DIR, TWIDDLE>(a);
    case 32: return launch_strided_t<32, DIR, TWIDDLE>(a);
    case 64: return launch_strided_t<64, DIR, TWIDDLE>(a);
    case 128: return launch_strided_t<128, DIR, TWIDDLE>(a);
    case 256: return launch_strided_t<256, DIR, TWIDDLE>(a);
    case 512: return launch_strided_t<512, DIR, TWIDDLE>(a);
    case 1024: return launch_strided_t<1024, DIR, TWIDDLE>(a);
    case 2048: return launch_strided_t<2048, DIR, TWIDDLE>(a);
    case 4096: return launch_strided_t<4096, DIR, TWIDDLE>(a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_strided(int n1, const StridedArgs& a) {
  if (a.dir < 0) return a.twiddle ? launch_strided_dir<-1, true>(n1, a) : launch_strided_dir<-1, false>(n1, a);
  return a.twiddle ? launch_strided_dir<1, true>(n1, a) : launch_strided_dir<1, false>(n1, a);
}

template <int N2, int DIR>
static hipError_t launch_row_t(const FourStepArgs& a) {
  constexpr int C = fourstep_tile(N2), T = N2 / lds_epth(N2);
  if (a.n1 % C) return hipErrorInvalidValue;
  const long long blocks = a.batch * (a.n1 / C);
  hipLaunchKernelGGL((fourstep_row_kernel<N2, DIR>), dim3((unsigned)blocks), dim3(C * T), 0,
                     a.stream, a.t_re, a.t_im, a.out_re, a.out_im, a.tw2, a.n1, a.batch, a.scale);
  return hipGetLastError();
}

template <int DIR>
static hipError_t launch_row_dir(const FourStepArgs& a) {
  switch (a.n2) {
    case 64: return launch_row_t<64, DIR>(a);
    case 128: return launch_row_t<128, DIR>(a);
    case 256: return launch_row_t<256, DIR>(a);
    case 512: return launch_row_t<512, DIR>(a);
    case 1024: return launch_row_t<1024, DIR>(a);
    case 2048: return launch_row_t<2048, DIR>(a);
    case 4096: return launch_row_t<4096, DIR>(a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fourstep(const FourStepArgs& a) {
  StridedArgs col{a.in_re, a.in_im, a.t_re, a.t_im, a.tw1, a.tw_lo, a.tw_hi, a.batch, a.n2,
                  a.lo_bits, (unsigned)((long long)a.n1 * a.n2 - 1), 1.0f, a.dir, true, a.stream};
  hipError_t e = launch_strided(a.n1, col);
  if (e != hipSuccess) return e;
  return a.dir < 0 ? launch_row_dir<-1>(a) : launch_row_dir<1>(a);
}

}  // namespace tfa
