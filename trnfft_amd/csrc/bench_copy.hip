// Measurement aid for bench.py (not part of the C ABI in include/trnfft_amd.h): a plain copy of two
// fp32 planes into two others -- the split re/im traffic pattern of the FFT kernels -- in a few
// access styles, so the bench can report the memory system's achievable rate for exactly the
// bytes a transform moves, measured in the same run.  Built into libtfa_copy.so.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

// UNR float4 per plane per thread, grid-strided; NTL / NTS: non-temporal loads / stores.
template <int UNR, bool NTL, bool NTS>
__global__ __launch_bounds__(256) void copy2_kernel(const f4* __restrict__ a, const f4* __restrict__ b,
                                                    f4* __restrict__ c, f4* __restrict__ d, long long n4) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (UNR - 1) * stride < n4; i += UNR * stride) {
    f4 x[UNR], y[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      x[u] = NTL ? __builtin_nontemporal_load(a + i + u * stride) : a[i + u * stride];
      y[u] = NTL ? __builtin_nontemporal_load(b + i + u * stride) : b[i + u * stride];
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      if (NTS) {
        __builtin_nontemporal_store(x[u], c + i + u * stride);
        __builtin_nontemporal_store(y[u], d + i + u * stride);
      } else {
        c[i + u * stride] = x[u];
        d[i + u * stride] = y[u];
      }
    }
  }
  for (; i < n4; i += stride) {
    c[i] = a[i];
    d[i] = b[i];
  }
}

// One contiguous stream: the same bytes as one plane pair, read from one buffer and written to
// another (the fastest plain copy of a transform's traffic on this part).
__global__ __launch_bounds__(256) void copy1_kernel(const f4* __restrict__ a, f4* __restrict__ c, long long n4) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n4) __builtin_nontemporal_store(__builtin_nontemporal_load(a + i), c + i);
}

template <int UNR, bool NTL, bool NTS>
hipError_t launch(const float* a, const float* b, float* c, float* d, long long n, hipStream_t s) {
  const long long n4 = n / 4;
  long long blocks = (n4 + 256LL * UNR - 1) / (256LL * UNR);
  if (blocks < 1) blocks = 1;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((copy2_kernel<UNR, NTL, NTS>), dim3((unsigned)blocks), dim3(256), 0, s,
                     reinterpret_cast<const f4*>(a), reinterpret_cast<const f4*>(b), reinterpret_cast<f4*>(c),
                     reinterpret_cast<f4*>(d), n4);
  return hipGetLastError();
}

}  // namespace

extern "C" {

// Number of access styles tfa_bench_copy2 offers.
int tfa_bench_copy2_variants(void) { return 4; }

// c[i] = a[i], d[i] = b[i] for i < n (n a multiple of 4, planes 16-byte aligned) on `stream`:
// variant 0 non-temporal loads and stores, 1 temporal loads with non-temporal stores, 2 temporal
// loads and stores, 3 non-temporal with four float4 per plane per thread.  Returns a hipError_t.
int tfa_bench_copy2(const float* a, const float* b, float* c, float* d, long long n, int variant, void* stream) {
  if (n < 0 || (n & 3) != 0) return (int)hipErrorInvalidValue;
  if (((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(c) |
        reinterpret_cast<uintptr_t>(d)) & 15) != 0)
    return (int)hipErrorInvalidValue;
  if (n == 0) return (int)hipSuccess;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (variant) {
    case 0: return (int)launch<1, true, true>(a, b, c, d, n, s);
    case 1: return (int)launch<1, false, true>(a, b, c, d, n, s);
    case 2: return (int)launch<1, false, false>(a, b, c, d, n, s);
    case 3: return (int)launch<4, true, true>(a, b, c, d, n, s);
    default: return (int)hipErrorInvalidValue;
  }
}

// c[i] = a[i] for i < n as one stream (n a multiple of 4, both 16-byte aligned) on `stream`,
// non-temporal float4 loads and stores.  Returns a hipError_t.
int tfa_bench_copy1(const float* a, float* c, long long n, void* stream) {
  if (n < 0 || (n & 3) != 0) return (int)hipErrorInvalidValue;
  if (((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(c)) & 15) != 0) return (int)hipErrorInvalidValue;
  if (n == 0) return (int)hipSuccess;
  const long long n4 = n / 4;
  const long long blocks = (n4 + 255) / 256;
  if (blocks > 0x7fffffffLL) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(copy1_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     reinterpret_cast<const f4*>(a), reinterpret_cast<f4*>(c), n4);
  return (int)hipGetLastError();
}

}  // extern "C"
