// Launch interfaces of the device kernels (host side) plus small device helpers shared by them.
#pragma once
#include <hip/hip_runtime.h>

#include "fft_device.h"

namespace tfa {

// Per-workgroup LDS budget of gfx950 (160 KiB per CU, all of it addressable by one workgroup).
constexpr long long kLdsBytes = 163840;
// Compute units of MI355X (8 XCDs x 32).
constexpr int kNumCUs = 256;

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).  Remap the
// linear block index so that consecutive tiles run on the same XCD at about the same time:
// tiles that share HBM cache lines then meet in one L2 instead of eight.
__device__ __forceinline__ long long xcd_tile_remap(long long i, long long g) {
  const long long per = g / 8;
  if (i >= per * 8) return i;
  return (i % 8) * per + i / 8;
}

// 32-bit form for grids below 2^31 workgroups (the launchers check): the tile index then divides
// in a few 32-bit operations instead of a 64-bit division sequence.
__device__ __forceinline__ unsigned xcd_tile_remap32(unsigned i, unsigned g) {
  const unsigned per = g / 8;
  if (i >= per * 8) return i;
  return (i % 8) * per + i / 8;
}

// Streaming (non-temporal) global accesses: every element of a batched transform is read once
// and written once, so it should not displace other lines in L2 / the Infinity Cache.
__device__ __forceinline__ float ld_stream(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void st_stream4(float* p, float4 v) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<f4v*>(p));
}
__device__ __forceinline__ float4 ld_stream4(const float4* p) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v r = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
  return make_float4(r.x, r.y, r.z, r.w);
}

// floor(n / d) and n % d for 0 <= n < 2^24 and rd = 1.0f / d (float reciprocal, one correction
// step: exact in that range)
__device__ __forceinline__ int divmod_small(int n, int d, float rd, int& r) {
  int q = (int)((float)n * rd);
  r = n - q * d;
  if (r < 0) {
    --q;
    r += d;
  } else if (r >= d) {
    ++q;
    r -= d;
  }
  return q;
}

// Thread layout of the batched LDS kernels for transform length N: T threads per transform,
// XF transforms per workgroup (c2c_threads(N) threads per workgroup), PADN LDS entries per
// transform (float2 when the exchange is interleaved, floats per plane otherwise; 1 when the
// transform needs no exchange).
template <int N, int E_ = c2c_epth(N), int THR = c2c_threads(N)>
struct C2cThreads {
  static constexpr int E = E_;
  static constexpr int T = N / E;
  static constexpr int XF = T >= THR ? 1 : THR / T;
  static constexpr int THREADS = XF * T;
  static constexpr LdsShape S = make_shape(N, E);
  static constexpr int PADN = S.npass > 1 ? lds_pad(N) : 1;
};

// Columns per workgroup for a strided (column) pass over transforms of length L: as wide as the
// LDS and the 1024-thread limit allow (wider tiles = longer contiguous HBM segments), at most 64.
__host__ __device__ constexpr int fourstep_tile(int l) {
  int c = 64;
  while (c > 1 && ((long long)c * (lds_pad(l) + 1) * 8 > kLdsBytes || c * (l / lds_epth(l)) > 1024)) c /= 2;
  return c;
}

struct C2cArgs {
  const float* in_re;
  const float* in_im;  // nullptr: real input (imaginary part zero)
  float* out_re;
  float* out_im;
  const float2* tw;
  long long batch;
  float scale;
  int dir;
  hipStream_t stream;
};
hipError_t launch_c2c_lds(int n, const C2cArgs& a);

struct StridedArgs {
  const float* in_re;
  const float* in_im;  // nullptr: real input
  float* out_re;       // may equal in_re (in place)
  float* out_im;
  const float2* tw;     // LDS-FFT table for length n1 (lds_epth layout)
  long long outer;   // independent (n1 x stride) blocks
  long long stride;  // element stride of the transformed axis = number of columns
  float scale;
  int dir;
  hipStream_t stream;
};
hipError_t launch_strided(int n1, const StridedArgs& a);

// Longest axis the single-pass strided kernel takes; longer power-of-two axes (up to 2^24) run
// as two or three strided passes (strided multi-pass four-step) through a workspace.
constexpr int kMaxStridedN = 4096;
// Shortest axis that runs the strided multi-pass path (n = 4096 as two passes of 64: its single
// pass fits only 4 columns per workgroup).
constexpr int kMinStridedMultiPassN = 4096;
// Axes of 2^kStridedThreePassLg and more use three factors (each <= 256: 64-column tiles).
constexpr int kStridedThreePassLg = 21;
// Smallest trailing stride of the strided multi-pass path: the last pass reads runs of `stride`
// floats, and below these strides the alternative measured faster: the transpose round trip
// above 4096 (2^22 x 2: 112 vs 167 us; 2^20 x 1: 35 vs 37 us; from 4 / 8 columns the strided
// passes win 1.3-1.8x), the single-pass strided kernel at 4096 (stride 4: 103 vs 159 us; from
// 16 columns the two passes win 1.16-1.38x, 4 x 4096 x 4096 629 -> 455 us).
__host__ __device__ constexpr long long strided_fs_min_stride(int npass, long long n) {
  return n <= 4096 ? 16 : npass >= 3 ? 8 : 4;
}
// Contiguous power-of-two lengths from 2^kContigThreePassLg run as the three-pass strided path
// with stride 1 (factors <= 256) instead of the two-pass four-step, whose 4096-point passes have
// 8-column tiles: 1 x 2^24 224 -> 199 us (inverse 227 -> 210, real input 207 -> 193).  At 2^23
// and below it measured no better or slower (1 x 2^23 91 -> 103 us, 4 x 2^22 173 -> 185,
// 8 x 2^21 145 -> 185): a third HBM pass costs more than the wider tiles gain.
constexpr int kContigThreePassLg = 24;
struct StridedFourStepArgs {
  const float* in_re;
  const float* in_im;  // nullptr: real input
  float* t_re;         // workspace, outer * n * stride floats each
  float* t_im;
  float* out_re;       // may equal in_re (the first pass reads all input before the last writes); not the workspace
  float* out_im;
  int npass;            // 2 or 3 factors, n = len[0] * ... * len[npass-1], each 64..4096
  int len[3];
  const float2* tw[3];  // LDS-FFT table of each factor (lds_epth layout)
  const float2* tw_lo;  // W_n^j, j < 2^lo_bits
  const float2* tw_hi;  // W_n^(j << lo_bits)
  int lo_bits;
  long long outer, stride;
  float scale;
  int dir;
  hipStream_t stream;
};
hipError_t launch_strided_fourstep(const StridedFourStepArgs& a);

struct FourStepArgs {
  const float* in_re;
  const float* in_im;  // nullptr: real input
  float* t_re;         // workspace, batch * n1 * n2 floats each (blocked layout, see the kernels)
  float* t_im;
  float* out_re;
  float* out_im;
  const float2* tw1;  // LDS-FFT table for length n1 (fourstep_epth layout)
  const float2* tw2;  // LDS-FFT table for length n2 (fourstep_epth layout)
  const float2* tw_lo;  // W_N^j, j < 2^lo_bits
  const float2* tw_hi;  // W_N^(j << lo_bits)
  int n1, n2, lo_bits;
  long long batch;
  float scale;
  int dir;
  hipStream_t stream;
};
hipError_t launch_fourstep(const FourStepArgs& a);

struct BluesteinArgs {
  const float* in_re;
  const float* in_im;  // nullptr: real input
  float* out_re;
  float* out_im;
  const float2* chirp;  // n entries, exp(sign*i*pi*k^2/n) with the angle rounded as in fp32
  const float2* hs;     // m entries, FFT_m(h) / m
  const float2* tw_f;   // LDS-FFT tables for length m, forward and inverse (fused path)
  const float2* tw_i;
  int n, m;
  long long batch;
  float scale;
  hipStream_t stream;
  // wrapped convolution length (fused path): m = 2n - 1 - wrap < 2n - 1, 0 < wrap <= kBlueWrapMax;
  // hs then holds the filter with its wrap colliding taps summed, and the kernel corrects the
  // 2 * wrap outputs they reach
  int wrap = 0;
};
hipError_t launch_bluestein_fused(int m, const BluesteinArgs& a);
// Largest wrap (2n - 1 - m) of the fused Bluestein kernel's wrapped-convolution lengths.
constexpr int kBlueWrapMax = 15;
// Two-level fused Bluestein kernel (lengths M = 4096, 8192: M / 512 wavefronts of 512 points per
// row): offset of the cross-wave twiddle rows in its tables, after the 512-point wave transform's
// table.
__host__ __device__ constexpr bool blue_2l(int m) { return m == 2048 || m == 4096 || m == 8192 || m == 16384; }
// its wave transform length B and elements per lane (16384 = 16 waves x 1024 points, 16 per lane;
// the others 512-point waves, 8 per lane), and the entry of its tables where the cross factors
// W_m^(n_b w) start (after the wave transform's table)
__host__ __device__ constexpr int blue_2l_b(int m) { return m == 16384 ? 1024 : 512; }
__host__ __device__ constexpr int blue_2l_e(int m) { return m == 16384 ? 16 : 8; }
__host__ __device__ constexpr int blue_2l_twoff(int m) { return m == 16384 ? 2048 : 1024; }

// Bluestein down a strided axis (x viewed as (outer, n, stride)), m <= kMaxStridedBlueM.
constexpr int kMaxStridedBlueM = 4096;
struct StridedBlueArgs {
  const float* in_re;
  const float* in_im;  // nullptr: real input
  float* out_re;       // may equal in_re (in place)
  float* out_im;
  const float2* chirp;  // n entries
  const float2* hs;     // FFT_m(h) / m, m entries
  const float2* tw_f;   // LDS-FFT tables for length m in the lds_epth(m) layout
  const float2* tw_i;
  long long outer, stride;
  int n;
  float scale;
  hipStream_t stream;
};
hipError_t launch_strided_bluestein(int m, const StridedBlueArgs& a);

// Split (transposed-domain four-step) Bluestein, m = m1 * m2 >= 16384.
struct BlueSplitArgs {
  const float* in_re;
  const float* in_im;  // nullptr: real input
  float* out_re;
  float* out_im;
  float* ws_re;  // workspace, batch * m floats per plane
  float* ws_im;
  const float2* chirp;  // n entries
  const float2* hp;     // m entries: H/m in transposed order, hp[k1*m2 + k2] = H[k1 + m1*k2] / m
  const float2* tw1f;   // LDS-FFT tables for m1 (lds_epth layout), forward / inverse
  const float2* tw1i;
  const float2* tw2f;   // LDS-FFT tables for m2 (c2c_epth layout), forward / inverse
  const float2* tw2i;
  const float2* lo;  // W_m^j, j < 2^lo_bits
  const float2* hi;  // W_m^(j << lo_bits)
  int lo_bits, n;
  long long batch;
  float scale;
  hipStream_t stream;
};
hipError_t launch_bluestein_split(int m1, int m2, const BlueSplitArgs& a);

struct StftArgs {
  const float* signal;  // (batch, length)
  const float* window;  // n_fft
  float* out_re;        // (batch, n_bins, n_frames)
  float* out_im;
  const float2* tw;  // LDS-FFT table for n_fft, forward
  int length, hop, pad, n_frames, n_bins;
  long long batch;
  float scale;
  hipStream_t stream;
  // non-power-of-two n_fft (Bluestein per frame, padded length m): tw above is the forward table
  // for m, these the inverse table, the chirp (n_fft) and the filter spectrum H/m (m)
  const float2* tw_i = nullptr;
  const float2* chirp = nullptr;
  const float2* hs = nullptr;
  int m = 0;
  // output planes (batch, n_frames, n_bins) instead of (batch, n_bins, n_frames)
  bool frames_major = false;
};
hipError_t launch_stft(int n_fft, const StftArgs& a);
hipError_t launch_stft_blue(int n_fft, const StftArgs& a);  // a.m != 0

struct RealArgs {
  const float* in_re;  // forward: (batch, n) real rows; inverse: (batch, n/2+1) bins
  const float* in_im;  // inverse only
  float* out_re;       // forward: (batch, n/2+1) bins; inverse: (batch, n) real rows
  float* out_im;       // forward only
  const float2* tw;    // LDS-FFT table for length n/2 in the plan's direction
  const float2* twr;   // W_n^k = exp(-2 pi i k / n), k < n/2
  long long batch;
  float scale;  // inverse: 1/n
  bool inverse;
  hipStream_t stream;
};
hipError_t launch_real(int n, const RealArgs& a);

struct IstftArgs {
  const float* spec_re;  // (batch, bins, n_frames), bins = n_fft/2+1 (n_fft when two_sided)
  const float* spec_im;
  const float* window;   // n_fft
  float* out;            // (batch, out_pitch)
  const float2* tw;      // inverse LDS-FFT table for n_fft (istft_epth layout)
  int n_frames, hop, halo;  // halo = floor((n_fft-1)/hop) frames recomputed before each tile
  long long batch;
  long long expected_len;  // n_fft + (n_frames-1)*hop samples before the centre trim
  long long start;         // first kept sample (n_fft/2 when centred)
  long long write_len;     // samples written per row; [write_len, out_pitch) is zero-filled
  long long out_pitch;
  float scale;  // 1/n_fft (x sqrt(n_fft) when normalized)
  hipStream_t stream;
  // adjoint of the forward STFT instead of its inverse: bins 0 and n_fft/2 count twice against
  // the others (scale 1/2 then gives the r2c adjoint), the windowed sum is written as it is (no
  // envelope division, no raw-sum branch)
  bool adjoint = false;
  // hop, start, out_pitch and write_len multiples of 4 and out 16-byte aligned: interior tiles
  // write four consecutive samples per thread (host-checked)
  bool vec4 = false;
  // input planes (batch, n_frames, bins) instead of (batch, bins, n_frames)
  bool frames_major = false;
  // two-sided spectra (bins = n_fft, power-of-two n_fft, not with `adjoint`): each frame is the
  // real part of its inverse transform; otherwise onesided (bins = n_fft/2 + 1)
  bool two_sided = false;
  // n_fft that is not a power of two (one inverse Bluestein chain per frame, length m): forward
  // and inverse m-point tables, the inverse chirp (n_fft) and its filter spectrum H/m (m)
  const float2* blue_tw_f = nullptr;
  const float2* blue_tw_i = nullptr;
  const float2* chirp = nullptr;
  const float2* hs = nullptr;
  int m = 0;
};
hipError_t launch_istft(int n_fft, const IstftArgs& a);
int istft_frames_per_tile(int n_fft, bool two_sided = false);
hipError_t launch_istft_blue(int n_fft, const IstftArgs& a);  // a.m != 0

struct Fft2Args {
  const float* in_re;
  const float* in_im;  // nullptr: real input
  float* out_re;       // must not alias the input
  float* out_im;
  const float2* tw_w;       // LDS-FFT table for length w (complex rows)
  const float2* tw_w_pair;  // LDS-FFT table for length w in the paired-real-row layout
  const float2* tw_hr;      // LDS-FFT table for length h/8 (column pass layout)
  const float2* tw_h;   // W_h^i, i < h
  const float2* tw_sw;  // single-pass small-image kernel: LDS-FFT tables for w and h
  const float2* tw_sh;  //   (fft2_small_epth layout); used when fft2_small_ok(h, w)
  long long batch, h, w;
  float scale;  // applied in pass 2 (1/(h*w) for the inverse)
  int dir;
  hipStream_t stream;
};
hipError_t launch_fft2(const Fft2Args& a);

// Operand ops of the complex GEMM: 0 = X, 1 = X^T, 2 = conj(X)^T, 3 = conj(X)
struct GemmArgs {
  long long m, n, k;
  const float* a_re;
  const float* a_im;
  long long lda;
  int a_op;
  const float* b_re;
  const float* b_im;
  long long ldb;
  int b_op;
  const float* bias_re;  // nullable
  const float* bias_im;
  float* c_re;
  float* c_im;
  long long ldc;
  float alpha;
  hipStream_t stream;
  long long batch = 1;            // matrix triples (grid.y)
  long long sa = 0, sb = 0, sc = 0;  // batch strides in floats (0: operand shared by the batch)
};
hipError_t launch_cgemm(const GemmArgs& a);

}  // namespace tfa
