// Strided four-step: a power-of-two axis of length N = N1*N2 > 4096 transformed where it lies,
// data viewed as (outer, N, S) row-major.  Position n = N2*n1 + n2, output k = k1 + N1*k2 (the
// split of the contiguous four-step), column s < S.  Two strided passes through a workspace, no
// transposes:
//   pass 1 (L = N1): columns col = n2*S + s of each outer block, element stride N2*S; DFT over n1,
//     times W_N^(n2*k1), written to tmp[o][k1][n2][s] (the input's own layout);
//   pass 2 (L = N2): columns col = k1*S + s; DFT over n2 read from tmp[o][k1][.][s] (element
//     stride S, base k1*N2*S + s), written to X[o][k1 + N1*k2][s] (element stride N1*S, base col).
// Replaces, for such axes, the transpose-copy + contiguous FFT + transpose-back of
// trnfft/api.py:496-516 (_fft_along_dim).
#include "kernels.h"

namespace tfa {

// One kernel serves both passes: column col = q*S + r (q = col / S) is read from
// o*blk + q*in_hi + r + j*in_step (j < L) and written to o*blk + q*out_hi + r + k*out_step.  A
// workgroup takes C adjacent columns of one outer block (the strided kernel's shape); with
// N1, N2 >= 64 >= C every tile is whole.  TWIDDLE (pass 1): output k1 of column col is
// multiplied by W_N^(q*k1), read as W^lo * W^hi from the two small tables.
template <int L, int DIR, bool REAL_IN, bool TWIDDLE, int C = fourstep_tile(L)>
__global__ __launch_bounds__(C * (L / lds_epth(L))) void strided_fs_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* __restrict__ out_re,
    float* __restrict__ out_im, const float2* __restrict__ tw, const float2* __restrict__ tw_lo,
    const float2* __restrict__ tw_hi, long long S, long long blk, long long in_hi, long long in_step,
    long long out_hi, long long out_step, long long tiles_per_block, int lo_bits, unsigned nmask, float scale) {
  constexpr int E = lds_epth(L), T = L / E;
  constexpr int PADN = lds_pad(L) + 1;
  // interleaved (re, im) exchange except at 4096 (as the single-pass strided kernel)
  constexpr bool IL = L != 4096;
  __shared__ float2 lds[C * PADN];
  const int c = threadIdx.x % C;  // column within the tile (fast across lanes)
  const int t = threadIdx.x / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long o = tile / tiles_per_block;
  const long long col = (tile % tiles_per_block) * C + c;
  const long long q = col / S, r = col - q * S;
  const size_t ib = (size_t)(o * blk + q * in_hi + r) + (size_t)t * (size_t)in_step;
  const size_t istep = (size_t)T * (size_t)in_step;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = ib + e * istep;
    v[e] = make_float2(ld_stream(in_re + i), REAL_IN ? 0.0f : ld_stream(in_im + i));
  }
  if constexpr (IL) {
    LdsFft<L, E, DIR, false, false, true>::run(v, reinterpret_cast<float*>(lds + c * PADN), nullptr, tw, t);
  } else {
    float* planes = reinterpret_cast<float*>(lds);
    LdsFft<L, E, DIR, false>::run(v, planes + c * PADN, planes + (C + c) * PADN, tw, t);
  }
  if constexpr (TWIDDLE) {
    // k1 = t + T*(TF*a + j): W^(q*(t + T*TF*a)) * W^(q*T*j), TF-1 + E/TF table pairs per thread
    constexpr int TF = E < 4 ? E : 4;
    const unsigned qq = (unsigned)q;
    const unsigned lomask = (1u << lo_bits) - 1;
    float2 w[TF];
#pragma unroll
    for (int j = 1; j < TF; ++j) {
      const unsigned m = (qq * (unsigned)(T * j)) & nmask;
      w[j] = cmul(tw_lo[m & lomask], tw_hi[m >> lo_bits]);
    }
#pragma unroll
    for (int a = 0; a < E / TF; ++a) {
      const unsigned m = (qq * (unsigned)(t + T * TF * a)) & nmask;
      const float2 p = cmul(tw_lo[m & lomask], tw_hi[m >> lo_bits]);
      v[TF * a] = cmul(v[TF * a], p);
#pragma unroll
      for (int j = 1; j < TF; ++j) v[TF * a + j] = cmul(v[TF * a + j], cmul(p, w[j]));
    }
  }
  const size_t ob = (size_t)(o * blk + q * out_hi + r) + (size_t)t * (size_t)out_step;
  const size_t ostep = (size_t)T * (size_t)out_step;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = ob + e * ostep;
    const float2 y = TWIDDLE ? v[e] : cscale(v[e], scale);
    if constexpr (C * 4 < 128) {
      // row segments shorter than a cache line: plain stores (L2 merges neighbouring partial lines)
      out_re[i] = y.x;
      out_im[i] = y.y;
    } else {
      st_stream(out_re + i, y.x);
      st_stream(out_im + i, y.y);
    }
  }
}

template <int N1, int N2, int DIR>
static hipError_t launch_strided_fs_t(const StridedFourStepArgs& a) {
  constexpr int C1 = fourstep_tile(N1), C2 = fourstep_tile(N2);
  constexpr int TH1 = C1 * (N1 / lds_epth(N1)), TH2 = C2 * (N2 / lds_epth(N2));
  static_assert(N2 % C1 == 0 && N1 % C2 == 0, "strided four-step tiles must be whole");
  const long long S = a.stride, N = (long long)N1 * N2, blk = N * S;
  const unsigned nmask = (unsigned)(N - 1);
  const long long tiles1 = (long long)N2 * S / C1, tiles2 = (long long)N1 * S / C2;
  if (a.outer * tiles1 > 0xffffffffLL || a.outer * tiles2 > 0xffffffffLL) return hipErrorInvalidValue;
  // pass 1: columns n2*S + s, element stride N2*S, same layout in and out, twiddled
  if (a.in_im == nullptr)
    hipLaunchKernelGGL((strided_fs_kernel<N1, DIR, true, true>), dim3((unsigned)(a.outer * tiles1)), dim3(TH1), 0,
                       a.stream, a.in_re, a.in_im, a.t_re, a.t_im, a.tw1, a.tw_lo, a.tw_hi, S, blk, S,
                       (long long)N2 * S, S, (long long)N2 * S, tiles1, a.lo_bits, nmask, 1.0f);
  else
    hipLaunchKernelGGL((strided_fs_kernel<N1, DIR, false, true>), dim3((unsigned)(a.outer * tiles1)), dim3(TH1), 0,
                       a.stream, a.in_re, a.in_im, a.t_re, a.t_im, a.tw1, a.tw_lo, a.tw_hi, S, blk, S,
                       (long long)N2 * S, S, (long long)N2 * S, tiles1, a.lo_bits, nmask, 1.0f);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // pass 2: columns k1*S + s, read at k1*N2*S + s + n2*S, written at k1*S + s + k2*N1*S
  hipLaunchKernelGGL((strided_fs_kernel<N2, DIR, false, false>), dim3((unsigned)(a.outer * tiles2)), dim3(TH2), 0,
                     a.stream, a.t_re, a.t_im, a.out_re, a.out_im, a.tw2, a.tw_lo, a.tw_hi, S, blk, (long long)N2 * S,
                     S, S, (long long)N1 * S, tiles2, a.lo_bits, nmask, a.scale);
  return hipGetLastError();
}

// n = n1 * n2 with n1 = 2^floor(lg/2) <= n2 (the plan's split)
template <int DIR>
static hipError_t launch_strided_fs_dir(const StridedFourStepArgs& a) {
  const long long key = (long long)a.n1 * 8192 + a.n2;
  switch (key) {
    case 64LL * 8192 + 128: return launch_strided_fs_t<64, 128, DIR>(a);
    case 128LL * 8192 + 128: return launch_strided_fs_t<128, 128, DIR>(a);
    case 128LL * 8192 + 256: return launch_strided_fs_t<128, 256, DIR>(a);
    case 256LL * 8192 + 256: return launch_strided_fs_t<256, 256, DIR>(a);
    case 256LL * 8192 + 512: return launch_strided_fs_t<256, 512, DIR>(a);
    case 512LL * 8192 + 512: return launch_strided_fs_t<512, 512, DIR>(a);
    case 512LL * 8192 + 1024: return launch_strided_fs_t<512, 1024, DIR>(a);
    case 1024LL * 8192 + 1024: return launch_strided_fs_t<1024, 1024, DIR>(a);
    case 1024LL * 8192 + 2048: return launch_strided_fs_t<1024, 2048, DIR>(a);
    case 2048LL * 8192 + 2048: return launch_strided_fs_t<2048, 2048, DIR>(a);
    case 2048LL * 8192 + 4096: return launch_strided_fs_t<2048, 4096, DIR>(a);
    case 4096LL * 8192 + 4096: return launch_strided_fs_t<4096, 4096, DIR>(a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_strided_fourstep(const StridedFourStepArgs& a) {
  if (a.stride < kMinStridedFourStepStride || a.outer < 1) return hipErrorInvalidValue;
  return a.dir < 0 ? launch_strided_fs_dir<-1>(a) : launch_strided_fs_dir<1>(a);
}

}  // namespace tfa
