// Compile-time shape of the LDS-resident Stockham FFT, shared by the device kernels and the
// host code that builds their twiddle tables (both must agree on pass order and table layout).
#pragma once
#include <hip/hip_runtime.h>

namespace tfa {

constexpr int kMaxPasses = 8;

__host__ __device__ constexpr int ilog2(long long n) {
  int l = 0;
  while ((1LL << l) < n) ++l;
  return l;
}

// Complex elements each thread keeps in registers for a length-N transform.  A transform of
// length N is handled by T = N / E threads; every pass but the last is radix E.  The choice per N
// comes from a launch-shape sweep of the batched kernel on MI355X (64 MiB per launch, buffers
// rotated past the Infinity Cache): 512 and 4096 are fastest at E = 32 (2 passes for 512),
// the other lengths at E = 16 (1024 = 16*16*4, 2048 = 16*16*8, 4 or 2 transforms per block).
__host__ __device__ constexpr int lds_epth(int n) {
  return n <= 16 ? n : (n == 32 || n == 64) ? 8 : (n == 512 || n == 4096) ? 32 : 16;
}

// Batched c2c kernel launch shape (elements per thread, threads per workgroup), from an in-run
// sweep on MI355X over E in {4, 8, 16, 32} and 256..1024 threads at 4M complex elements per
// launch, buffers rotated past the Infinity Cache.  Headline N = 1024: E = 8 / 512 threads,
// 13.12 us against 13.64 us for the former E = 16 / 256.  Other lengths (us, new vs former):
// 128 14.8 vs ~16, 256 14.2 vs ~15, 4096 14.2 vs 16.5, 8192 16.2 vs 19.0, 16384 22.3 vs 24.6;
// 512 and 2048 unchanged within 1 %.  n <= 64 run the staged short-row kernel with n / c2c_epth
// threads per row: E = 8 there (n = 16: 14.9 -> 12.6 us, 64: 15.6 -> 12.6 us against E = 16 / 4).
__host__ __device__ constexpr int c2c_epth(int n) {
  return n == 16 || n == 64 ? 8 : n == 128 ? 4 : (n == 256 || n == 1024 || n == 2048 || n == 4096) ? 8
         : (n == 8192 || n == 16384) ? 32 : lds_epth(n);
}
// Interleaved (re, im) LDS exchange (one 64-bit access per element) in the batched c2c kernel:
// measured 1-4 % faster at most lengths (identical results), 2-4 % slower at 512 and 8192.
// (The exchange one plane at a time, half the LDS per row, measured slower from 2048 up: 8192
// 15.4 -> 16.6 us, 16384 18.5 -> 20.5 at 4M points.)
__host__ __device__ constexpr bool c2c_il(int n) { return n != 512 && n != 8192; }
// Next-pass twiddle prefetch (LdsFft PF) where one or two transforms fill a workgroup and the
// table latency after each exchange is exposed: N = 16384 21.2 -> 18.8 us; at high occupancy it
// costs registers and time (N = 1024: 12.7 -> 15.3 us), so it is off below 8192.
__host__ __device__ constexpr bool c2c_pf(int n) { return n >= 8192; }
__host__ __device__ constexpr int c2c_threads(int n) {
  return n == 64 || n == 256 ? 1024 : (n == 128 || n == 1024 || n == 2048 || n == 4096 || n == 16384) ? 512 : 256;
}

// Elements per thread of the real-row kernels (r2c / c2r over a half-length h complex transform),
// from a launch-shape sweep on MI355X (4M real samples per launch, buffers rotated past the
// Infinity Cache): small transforms want E = 4 (more lanes per row segment), mid sizes E = 8
// (one wavefront per transform up to h = 512), the largest E = 32 (fewest workgroup barriers).
__host__ __device__ constexpr int real_epth(int h, bool inverse) {
  return h <= 2 ? h : h >= 8192 ? 32 : (h <= (inverse ? 64 : 256)) ? 4 : 8;
}
// next-pass twiddle prefetch for the real-row kernels where a workgroup holds one row (h >= 8192)
__host__ __device__ constexpr bool real_pf(int h) { return h >= 8192; }

// Elements per thread of the forward STFT's pair transforms (many lanes per transform measured
// fastest at every n_fft).
__host__ __device__ constexpr int stft_epth(int n) { return n < 8 ? n : 8; }
// next-pass twiddle prefetch in the STFT transforms from n_fft = 1024 (8 or fewer pairs per
// workgroup: n_fft 1024 84 -> 77 us; at 512 it measured 1 % slower)
__host__ __device__ constexpr bool stft_pf(int n) { return n >= 1024; }
// Dynamic LDS (bytes, unused by the kernel) added to the STFT launch to hold it to one 1024-thread
// workgroup per CU: at n_fft = 512 (64 x 160000 samples, hop 256) one workgroup per CU measured
// 39.5 us against 43.3 us for two (the output's bin-row segments reach HBM in a better order).
__host__ __device__ constexpr unsigned stft_lds_extra(int n) { return n == 512 ? 16384u : 0u; }

// Elements per thread of the 2-D transform's paired real-row pass 1 and column pass 2 (the
// many-lanes-per-transform shape that also won for the STFT).
__host__ __device__ constexpr int fft2_pair_epth(int w) { return w < 8 ? w : w >= 4096 ? 16 : 8; }
__host__ __device__ constexpr int fft2_col_epth(int hr) { return hr < 8 ? hr : 8; }

// Single-pass 2-D transform of small images (h*w <= 16384 complex: whole images in LDS).  A
// workgroup of 1024 threads takes IMG images (4096 elements when images are smaller) and keeps
// E = IMG*h*w/1024 elements per thread in both the row and the column phase.
__host__ __device__ constexpr int fft2_small_img(int h, int w) { return h * w >= 4096 ? 1 : 4096 / (h * w); }
__host__ __device__ constexpr int fft2_small_epth(int h, int w) { return fft2_small_img(h, w) * h * w / 1024; }
__host__ __device__ constexpr bool fft2_small_ok(long long h, long long w) {
  return h >= 4 && w >= 4 && (h & (h - 1)) == 0 && (w & (w - 1)) == 0 && h * w <= 16384 &&
         h >= fft2_small_epth((int)h, (int)w) && w >= fft2_small_epth((int)h, (int)w);
}

// Fused Bluestein launch shape, from in-run A/B sweeps on MI355X with the next-pass twiddle
// prefetch on.  E = 8 elements per thread for m = 128..8192: more lanes per row (a row per
// workgroup from m = 512 at 256/512 threads, 1024 at m = 8192) and ~90 VGPRs, against E = 16/32
// with 100-244: m = 128 7.2 -> 4.8 us (1024 rows), 256 8.2 -> 5.2, 512 17.0 -> 6.1, 1024 11.5 ->
// 8.6, 4096 (256 rows) 23.1 -> 9.3, 8192 (256 rows) 27.6 -> 14.7; m = 16384 (256 x 4099) E = 16 with
// 1024 threads, 31.7 -> 29.5 us against E = 32 / 512.  The prefetch pays from m = 256 (every
// workgroup runs the same pass at the same time, so each pass's table latency is exposed): C3a
// 1024 x 1000 12.9 -> 12.3 us.  (Twiddle tables staged in LDS once per workgroup measured
// slower, C3a 13.0 -> 17.0 us: the 41 KB copy costs more than it saves.)
// Mixed-radix length 9216 = 12 * 12 * 4 * 4 * 4 (4104 < n <= 4608; measured at n = 4099, 256 rows, before
// the wrapped 8192-point length took that n over): E = 12 with 768 threads per row
// measured 18.2 us against 22.6 us for E = 24 / 384 threads (181 VGPRs), 24.9 us for E = 24 forced
// to two workgroups per CU and 26.7 us for E = 24 without the twiddle prefetch (the former
// power-of-two m = 16384 kernel: 29.0 us).  Timing probes of that kernel: the LDS exchanges cost
// 3.5 us and the twiddle-table reads 1.4 us of the 18.9; the rest is VALU (1536 instructions per
// wave, each 4 cycles on a 16-lane SIMD) and the load latencies.
// Mixed-radix lengths 3 * 2^k below that, measured against the power-of-two length the reference
// pads to (4M complex elements per launch; only the faster ones are used):
// 768 (E = 12, 256 threads) n = 300: 45.3 against 59.8 us at 1024, n = 380: 39.2 against 50.3;
// 1536 (E = 24, 256 threads) n = 600: 57.7 against 62.4 at 2048, n = 700: 46.1 against 55.3;
// 3072 (E = 12, 256 threads) n = 1300: 57.6 against 62.6 at 4096, n = 1500: 52.0 against 55.2;
// 12288 (E = 24, 512 threads, 24 x 8^3, 191 VGPRs) n = 5000 x 838: 69.0 against 102.5 at 16384.
// Slower or no better: 6144 as 24 x 16^2 (E = 24, 256 threads) against the two-level kernel at
// 8192 (n = 3000 x 1398 72.6 against 51.6 us, 16 rows 12.7 against 8.8), 96, 192, 384 (within 3 %), 6144 (84 against 79 us at 8192), E = 12 with
// 512 threads at 1536 and 3072 (70-79 us), E = 6 at 768 (65-89 us).  The plan takes these lengths
// (blue_fused_length) only where they hold 2n - 1 points and are shorter than m.
__host__ __device__ constexpr int blue_epth(int m) {
  return m == 1536 || m == 12288 ? 24 : m % 3 == 0 ? 12 : m >= 16384 ? 16 : m >= 128 ? 8 : lds_epth(m);
}
__host__ __device__ constexpr int blue_threads(int m) {
  return m % 3 == 0 ? (m == 9216 ? m / 12 : 256) : m == 2048 || m >= 8192 ? 512 : 256;
}
__host__ __device__ constexpr bool blue_pf(int m) { return m >= 256; }
// double-buffered LDS exchange in the fused kernel (one barrier per pass exchange) where two
// buffers fit the CU's LDS: C3a (m = 2048) 12.8 -> 12.2 us; no change at m = 9216
__host__ __device__ constexpr bool blue_db(int m) { return (m % 3 == 0 && m <= 9216) || (m >= 1024 && m <= 8192); }
// wrapped-convolution lengths of the fused kernel (power-of-two M = 2n - 1 - wrap, 1 <= wrap <= 15):
// from 128 (16 threads per row, so the corrected outputs k < wrap are all in element 0)
__host__ __device__ constexpr bool blue_wrap_ok(int m) { return m >= 128 && m <= 16384 && (m & (m - 1)) == 0; }
// split Bluestein (m >= 32768, three passes): elements per thread of the column passes (length
// m1; E = 8 at m1 = 128 measured no better) and next-pass twiddle prefetch in the column and row
// passes (209 x 20000 147 -> 143 us, 59 x 70000 183 -> 178, 32 x 8193 26.9 -> 25.7; 511 x 8193
// 1 % slower)
__host__ __device__ constexpr int blue_col_epth(int m1) { return lds_epth(m1); }
__host__ __device__ constexpr bool blue_split_pf(int) { return true; }

// Inverse-STFT launch shape from a sweep on MI355X (64 x 160000 samples, hop n/2, n_fft 16..4096,
// E in {4, 8, 16} x 128..1024 threads): E = 8 elements per thread up to n = 2048, 16 at 4096;
// 256 threads per workgroup up to n = 64, 512 up to 1024, 1024 above (n = 16: 64 -> 45 us,
// 256: 65 -> 48, 1024: 73 -> 63, 4096: 122 -> 100 against the former shapes).  With frames-major
// spectra (in-run A/B, hop n/2): n = 256 at 256 threads 30.2 -> 29.2 us; n = 1024 at 1024 threads
// 36.7 -> 42.8 (kept at 512); E = 16 at 1024 / 2048 38.2 -> 43.8 / 42.2 -> 55.9 us (kept at 8).
__host__ __device__ constexpr int istft_epth(int n) { return n <= 2048 ? 8 : 16; }
__host__ __device__ constexpr int istft_threads(int n) { return n <= 64 || n == 256 ? 256 : n <= 1024 ? 512 : 1024; }
// next-pass twiddle prefetch in the inverse STFT from n_fft = 512 (C2's inverse 53.4 -> 52.6 us,
// n_fft 1024 127 -> 122)
__host__ __device__ constexpr bool istft_pf(int n) { return n >= 512; }

// Elements per thread of the four-step passes over transforms of length l (128..4096): 32 threads
// per transform up to l = 1024 (one 32-transform tile = 1024 threads), 32 elements above.
__host__ __device__ constexpr int fourstep_epth(int l) { return l <= 1024 ? (l >= 128 ? l / 32 : 4) : 32; }

__host__ __device__ constexpr int gcd_c(int a, int b) {
  while (b) {
    const int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

struct LdsShape {
  int n, e, t, npass;
  int radix[kMaxPasses];
  int ls[kMaxPasses];       // product of the radices of the earlier passes
  int twoff[kMaxPasses + 1];  // offset (in complex entries) of each pass's twiddle block
};

// Pass p (p >= 1) multiplies input r of a butterfly with in-transform position k (k < ls[p])
// by W_{ls[p]*radix[p]}^{r*k}; its block holds ls[p] rows of radix[p] entries (entry r = 0 is 1).
__host__ __device__ constexpr LdsShape make_shape(int n, int e) {
  LdsShape s{};
  s.n = n;
  s.e = e;
  s.t = n / e;
  int rem = n, p = 0, ls = 1, off = 0;
  while (rem > 1) {
    // the largest radix dividing both the remaining length and E (E itself while it divides; for
    // powers of two this is min(E, rem))
    int r = gcd_c(e, rem);
    if (r <= 1) r = rem;  // no common factor: one pass of the rest (rejected by the device code)
    s.radix[p] = r;
    s.ls[p] = ls;
    s.twoff[p] = off;
    if (p > 0) off += ls * r;
    ls *= r;
    rem /= r;
    ++p;
  }
  s.npass = p;
  s.twoff[p] = off;
  return s;
}

// LDS word index with one pad word per 16 to keep the strided pass writes bank-conflict free.
__host__ __device__ constexpr int lds_pad(int i) { return i + (i >> 4); }

// Non-power-of-two STFT: one Bluestein transform of length m per frame, m a power of two
// (32..4096) or 3 * 2^k (96..3072), the shortest with n + n_bins - 1 <= m.
constexpr int kStftBlueMinM = 32;
constexpr int kStftBlueMaxM = 4096;
__host__ __device__ constexpr bool stft_blue_len_ok(long long m) {
  if (m < kStftBlueMinM || m > kStftBlueMaxM) return false;
  const long long q = m % 3 == 0 ? m / 3 : m;
  return q >= 32 && (q & (q - 1)) == 0;
}
// largest n_fft a length-m transform serves (onesided: n + n/2 <= m)
__host__ __device__ constexpr int stft_blue_nmax(int m) {
  int n = 2 * m / 3 + 2;
  while (n + n / 2 > m) --n;
  return n;
}
// Launch shape (elements per thread, frames per workgroup) from a sweep on MI355X (64 x 160000
// samples, hop 2n/5, every E in {4..32} dividing m and 2..64 frames per workgroup; the kernel is
// VALU-bound, ~1 wavefront-instruction per 64 points per pass): n_fft 30 (m 64) 128 us, 100 (192)
// 148, 200 (384) 177, 257 (512) 177, 400 (768) 186, 600 (1024) 188, 1000 (1536) 199, 1300 (2048)
// 187, 2000 (3072) 232.  (m = 1024 at E = 16 / 16 frames, the first shape: 270 us for n_fft 400;
// the shortest-length rule with the truncated filter took n_fft 400 from 1024 to 768 points,
// 320 from 1024 to 512 and 600 from 2048 to 1024.)
__host__ __device__ constexpr int stft_blue_epth(int m) {
  return (m == 384 || m == 768 || m == 1536) ? 24 : m % 3 == 0 ? 12 : 8;
}
__host__ __device__ constexpr int stft_blue_frames(int m) {
  return m <= 32 ? 32 : m <= 512 ? 16 : m <= 1024 ? 8 : m <= 2048 ? 4 : 2;
}
// Floats of LDS per frame: the exchange buffer of the m-point transform (its spectrum, at most
// m/2 float2, is staged there afterwards), rounded so that successive frames start g banks apart,
// g = 128 / frames: the output stage reads bin k of `frames` consecutive frames per instruction.
__host__ __device__ constexpr int stft_blue_area(int m, int frames) {
  const int g = frames >= 32 ? 4 : (128 / frames) % 64;
  int a = 2 * lds_pad(m);
  while (a % 64 != g) a += 4;
  return a;
}
// Inverse STFT at n_fft that is not a power of two (one inverse Bluestein chain per frame, m >=
// 2n - 1 since every sample of a frame is kept): elements per thread and frames per workgroup
// (owned frames + the recomputed halo of floor((n-1)/hop) frames; up to 1024 threads within the
// LDS, which also holds the window).  Measured on MI355X (64 signals, 160000 output samples):
// n_fft 400 / hop 160 (m 1024) E = 16 with 16 frames 321 us against 355 for E = 8 with 8 and 336
// for E = 32 with 16 (hop 100: 526 / 649 / 559); n_fft 320 (m 768) E = 12 with 8 frames 219 us
// against 229-258 for the others; n_fft 1000 / hop 250 (m 2048) E = 16 with 8 frames 662 us
// against 711 for E = 32 (fewer frames per workgroup recompute more halo: 1348-1660).
__host__ __device__ constexpr int istft_blue_epth(int m) {
  return m == 768 ? 12 : m % 3 == 0 ? stft_blue_epth(m) : m >= 1024 ? 16 : 8;
}
__host__ __device__ constexpr int istft_blue_frames(int m) {
  int f = m == 768 ? 8 : 1024 / (m / istft_blue_epth(m));
  f = f > 64 ? 64 : f < 1 ? 1 : f;
  while (f > 1 && f * stft_blue_area(m, f) * 4 + m * 2 > 160 * 1024) f /= 2;
  return f;
}
// The forward STFT's signal gradient at such n_fft (the inverse kernel's tiling on the forward
// plan's length and elements per thread): frames per workgroup, up to 1024 threads within the LDS
// (which holds the window of up to stft_blue_nmax(m) samples).
__host__ __device__ constexpr int stft_blue_adj_frames(int m) {
  int f = 1024 / (m / stft_blue_epth(m));
  f = f > 64 ? 64 : f < 1 ? 1 : f;
  while (f > 1 && f * stft_blue_area(m, f) * 4 + stft_blue_nmax(m) * 4 > 160 * 1024) f /= 2;
  return f;
}

}  // namespace tfa
