// Batched power-of-two complex-to-complex FFT kernels.
//
//  * c2c_lds_kernel: one launch per batch; each transform of length N <= 16384 stays in
//    registers + LDS for all its passes (replaces the reference's per-stage launches,
//    trnfft/fft_core.py:53-117 on CPU and :1063-1238 on the NKI path).
//  * fourstep_col_kernel / fourstep_row_kernel: N = N1*N2 > 16384 in two HBM passes
//    (column FFTs with the W_N^{n2*k1} twiddle fused into their store, then row FFTs whose
//    output is transposed through LDS so the strided store stays coalesced).  This is the
//    single-GPU form of the reference's row-column decomposition, trnfft/nki/multicore.py:151-219.
#include "kernels.h"

namespace tfa {

// ---------------------------------------------------------------------------------------------
// LDS-resident batched transform
// ---------------------------------------------------------------------------------------------
template <int N, int DIR, bool REAL_IN>
__global__ __launch_bounds__(C2cThreads<N>::THREADS) void c2c_lds_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re,
    float* out_im, const float2* __restrict__ tw, long long batch, float scale) {
  using C = C2cThreads<N>;
  constexpr int E = C::E, T = C::T;
  __shared__ float lre[C::XF * C::PADN];
  __shared__ float lim[C::XF * C::PADN];
  const int tid = threadIdx.x & (T - 1);
  const int xf = threadIdx.x / T;
  const long long b = (long long)blockIdx.x * C::XF + xf;
  const bool valid = b < batch;
  const size_t base = (size_t)b * N;

  float2 v[E];
  if (valid) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const size_t i = base + tid + T * e;
      v[e] = make_float2(in_re[i], REAL_IN ? 0.0f : in_im[i]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = make_float2(0.0f, 0.0f);
  }
  LdsFft<N, E, DIR, (T <= 64)>::run(v, lre + xf * C::PADN, lim + xf * C::PADN, tw, tid);
  if (valid) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const size_t i = base + tid + T * e;
      out_re[i] = v[e].x * scale;
      out_im[i] = v[e].y * scale;
    }
  }
}

template <int N, int DIR, bool REAL_IN>
static hipError_t launch_c2c_lds_t(const C2cArgs& a) {
  using C = C2cThreads<N>;
  const long long blocks = (a.batch + C::XF - 1) / C::XF;
  hipLaunchKernelGGL((c2c_lds_kernel<N, DIR, REAL_IN>), dim3((unsigned)blocks), dim3(C::THREADS),
                     0, a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.tw, a.batch, a.scale);
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
// Columns per workgroup for a strided pass over transforms of length L: as wide as the LDS and
// the 1024-thread limit allow (wider tiles = longer contiguous HBM segments), at most 64.
__host__ __device__ constexpr int fourstep_tile(int l) {
  int c = 64;
  while (c > 1 && ((long long)c * (lds_pad(l) + 1) * 8 > kLdsBytes || c * (l / lds_epth(l)) > 1024)) c /= 2;
  return c;
}

// Column pass: FFT over n1 of each column n2 (stride N2), times W_N^{n2*k1}, stored in place
// layout tmp[k1*N2 + n2].  One workgroup = C adjacent columns of one batch entry.
template <int N1, int DIR, bool REAL_IN>
__global__ __launch_bounds__(fourstep_tile(N1) * (N1 / lds_epth(N1))) void fourstep_col_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* __restrict__ t_re,
    float* __restrict__ t_im, const float2* __restrict__ tw, const float2* __restrict__ tw_lo,
    const float2* __restrict__ tw_hi, int n2_len, int lo_bits, long long batch) {
  constexpr int E = lds_epth(N1), T = N1 / E, C = fourstep_tile(N1);
  constexpr int PADN = lds_pad(N1) + 1;
  __shared__ float lre[C * PADN];
  __shared__ float lim[C * PADN];
  const int c = threadIdx.x % C;  // column within tile (fast across lanes: coalesced)
  const int t = threadIdx.x / C;
  const int tiles_per_row = n2_len / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long b = tile / tiles_per_row;
  const int n2 = (int)(tile % tiles_per_row) * C + c;
  const size_t N = (size_t)N1 * n2_len;
  const size_t base = (size_t)b * N + n2;

  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = base + (size_t)(t + T * e) * n2_len;
    v[e] = make_float2(in_re[i], REAL_IN ? 0.0f : in_im[i]);
  }
  LdsFft<N1, E, DIR, false>::run(v, lre + c * PADN, lim + c * PADN, tw, t);
  const unsigned nmask = (unsigned)(N - 1);
  const unsigned lomask = (1u << lo_bits) - 1;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int k1 = t + T * e;
    const unsigned m = ((unsigned)n2 * (unsigned)k1) & nmask;
    const float2 w = cmul(tw_lo[m & lomask], tw_hi[m >> lo_bits]);
    const float2 y = cmul(v[e], w);
    const size_t i = base + (size_t)k1 * n2_len;
    t_re[i] = y.x;
    t_im[i] = y.y;
  }
  (void)batch;
}

// Row pass: FFT over n2 of each row k1 of tmp (contiguous), output X[k1 + N1*k2] for C
// adjacent rows, transposed through LDS so each store covers C consecutive k1.
template <int N2, int DIR>
__global__ __launch_bounds__(fourstep_tile(N2) * (N2 / lds_epth(N2))) void fourstep_row_kernel(
    const float* __restrict__ t_re, const float* __restrict__ t_im, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, int n1_len, long long batch,
    float scale) {
  constexpr int E = lds_epth(N2), T = N2 / E, C = fourstep_tile(N2);
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

template <int N1, int DIR>
static hipError_t launch_col_t(const FourStepArgs& a, bool real_in) {
  constexpr int C = fourstep_tile(N1), T = N1 / lds_epth(N1);
  if (a.n2 % C) return hipErrorInvalidValue;
  const long long blocks = a.batch * (a.n2 / C);
  if (real_in)
    hipLaunchKernelGGL((fourstep_col_kernel<N1, DIR, true>), dim3((unsigned)blocks), dim3(C * T), 0,
                       a.stream, a.in_re, a.in_im, a.t_re, a.t_im, a.tw1, a.tw_lo, a.tw_hi, a.n2,
                       a.lo_bits, a.batch);
  else
    hipLaunchKernelGGL((fourstep_col_kernel<N1, DIR, false>), dim3((unsigned)blocks), dim3(C * T), 0,
                       a.stream, a.in_re, a.in_im, a.t_re, a.t_im, a.tw1, a.tw_lo, a.tw_hi, a.n2,
                       a.lo_bits, a.batch);
  return hipGetLastError();
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
static hipError_t launch_col_dir(const FourStepArgs& a, bool real_in) {
  switch (a.n1) {
    case 64: return launch_col_t<64, DIR>(a, real_in);
    case 128: return launch_col_t<128, DIR>(a, real_in);
    case 256: return launch_col_t<256, DIR>(a, real_in);
    case 512: return launch_col_t<512, DIR>(a, real_in);
    case 1024: return launch_col_t<1024, DIR>(a, real_in);
    case 2048: return launch_col_t<2048, DIR>(a, real_in);
    case 4096: return launch_col_t<4096, DIR>(a, real_in);
    default: return hipErrorInvalidValue;
  }
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
  const bool real_in = a.in_im == nullptr;
  hipError_t e = a.dir < 0 ? launch_col_dir<-1>(a, real_in) : launch_col_dir<1>(a, real_in);
  if (e != hipSuccess) return e;
  return a.dir < 0 ? launch_row_dir<-1>(a) : launch_row_dir<1>(a);
}

}  // namespace tfa
