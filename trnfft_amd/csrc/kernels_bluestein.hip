// Bluestein (chirp-z) transform for arbitrary n, trnfft/fft_core.py:1285-1376.
//
// Fused path (padded length m <= 16384): one launch, one row per transform slot.  The row is
// loaded, multiplied by the chirp and zero-padded in registers, transformed forward in LDS,
// multiplied by the plan's filter spectrum H/m, transformed back, multiplied by the chirp and
// stored (first n entries only): one HBM read and one HBM write per element, against the
// reference's three separate m-point FFTs and five full-size temporaries.
//
// Staged path (m > 16384): chirp/pad kernel -> four-step FFT_m -> pointwise * H/m -> four-step
// IFFT_m -> chirp/slice kernel, with the intermediate rows in the caller's workspace.
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
};

template <int M, bool REAL_IN, int E_ = blue_epth(M), int THR = blue_threads(M)>
__global__ __launch_bounds__((BlueCfg<M, E_, THR>::THREADS)) void bluestein_fused_kernel(
    const float* __restrict__ in_re, const float* __restrict__ in_im, float* out_re,
    float* out_im, const float2* __restrict__ chirp, const float2* __restrict__ hs,
    const float2* __restrict__ tw_f, const float2* __restrict__ tw_i, int n, long long batch,
    float scale) {
  using C = BlueCfg<M, E_, THR>;
  constexpr int E = C::E, T = C::T;
  __shared__ float lre[C::XF * C::PADN];
  __shared__ float lim[C::XF * C::PADN];
  const int tid = threadIdx.x & (T - 1);
  const int xf = threadIdx.x / T;
  const long long b = (long long)blockIdx.x * C::XF + xf;
  const bool valid = b < batch;
  const size_t base = (size_t)b * n;

  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid + T * e;
    float2 y = make_float2(0.0f, 0.0f);
    if (valid && i < n) {
      const float2 x = make_float2(in_re[base + i], REAL_IN ? 0.0f : in_im[base + i]);
      y = cmul(x, chirp[i]);
    }
    v[e] = y;
  }
  float* my_re = lre + xf * C::PADN;
  float* my_im = lim + xf * C::PADN;
  LdsFft<M, E, -1, (T <= 64)>::run(v, my_re, my_im, tw_f, tid);
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = cmul(v[e], hs[tid + T * e]);
  LdsFft<M, E, 1, (T <= 64)>::run(v, my_re, my_im, tw_i, tid);
  if (valid) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = tid + T * e;
      if (i < n) {
        const float2 y = cmul(v[e], chirp[i]);
        out_re[base + i] = y.x * scale;
        out_im[base + i] = y.y * scale;
      }
    }
  }
}

template <int M>
static hipError_t launch_blue_m(const BluesteinArgs& a) {
  using C = BlueCfg<M, blue_epth(M), blue_threads(M)>;
  const long long blocks = (a.batch + C::XF - 1) / C::XF;
  if (a.in_im == nullptr)
    hipLaunchKernelGGL((bluestein_fused_kernel<M, true>), dim3((unsigned)blocks), dim3(C::THREADS), 0,
                       a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.chirp, a.hs, a.tw_f, a.tw_i,
                       a.n, a.batch, a.scale);
  else
    hipLaunchKernelGGL((bluestein_fused_kernel<M, false>), dim3((unsigned)blocks), dim3(C::THREADS),
                       0, a.stream, a.in_re, a.in_im, a.out_re, a.out_im, a.chirp, a.hs, a.tw_f,
                       a.tw_i, a.n, a.batch, a.scale);
  return hipGetLastError();
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
    default: return hipErrorInvalidValue;
  }
}

// ---- staged path helpers ----------------------------------------------------------------------
// y[b, i] = x[b, i] * chirp[i] for i < n, 0 for n <= i < m.
__global__ void bluestein_pre_kernel(const float* __restrict__ in_re, const float* __restrict__ in_im,
                                     float* __restrict__ y_re, float* __restrict__ y_im,
                                     const float2* __restrict__ chirp, int n, int m, long long total) {
  const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= total) return;
  const long long b = g / m;
  const int i = (int)(g - b * m);
  float2 y = make_float2(0.0f, 0.0f);
  if (i < n) {
    const size_t s = (size_t)b * n + i;
    y = cmul(make_float2(in_re[s], in_im ? in_im[s] : 0.0f), chirp[i]);
  }
  y_re[g] = y.x;
  y_im[g] = y.y;
}

// y[b, i] *= hs[i]
__global__ void bluestein_mul_kernel(float* __restrict__ y_re, float* __restrict__ y_im,
                                     const float2* __restrict__ hs, int m, long long total) {
  const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= total) return;
  const int i = (int)(g % m);
  const float2 y = cmul(make_float2(y_re[g], y_im[g]), hs[i]);
  y_re[g] = y.x;
  y_im[g] = y.y;
}

// out[b, i] = y[b, i] * chirp[i] * scale for i < n
__global__ void bluestein_post_kernel(const float* __restrict__ y_re, const float* __restrict__ y_im,
                                      float* out_re, float* out_im, const float2* __restrict__ chirp,
                                      int n, int m, long long total, float scale) {
  const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= total) return;
  const long long b = g / n;
  const int i = (int)(g - b * n);
  const size_t s = (size_t)b * m + i;
  const float2 y = cmul(make_float2(y_re[s], y_im[s]), chirp[i]);
  out_re[g] = y.x * scale;
  out_im[g] = y.y * scale;
}

static unsigned blocks_for(long long total, int threads) {
  return (unsigned)((total + threads - 1) / threads);
}

hipError_t launch_bluestein_pre(const BluesteinArgs& a, float* y_re, float* y_im) {
  const long long total = a.batch * (long long)a.m;
  hipLaunchKernelGGL(bluestein_pre_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, a.stream,
                     a.in_re, a.in_im, y_re, y_im, a.chirp, a.n, a.m, total);
  return hipGetLastError();
}

hipError_t launch_bluestein_mul(const BluesteinArgs& a, float* y_re, float* y_im) {
  const long long total = a.batch * (long long)a.m;
  hipLaunchKernelGGL(bluestein_mul_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, a.stream,
                     y_re, y_im, a.hs, a.m, total);
  return hipGetLastError();
}

hipError_t launch_bluestein_post(const BluesteinArgs& a, const float* y_re, const float* y_im) {
  const long long total = a.batch * (long long)a.n;
  hipLaunchKernelGGL(bluestein_post_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, a.stream,
                     y_re, y_im, a.out_re, a.out_im, a.chirp, a.n, a.m, total, a.scale);
  return hipGetLastError();
}

}  // namespace tfa
