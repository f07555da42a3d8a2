// Host side of the C ABI (include/trnfft_amd.h): plan construction (algorithm choice and device
// tables), workspace sizing and execution dispatch.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <complex>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/trnfft_amd.h"
#include "kernels.h"

using tfa::LdsShape;

// Scratch of the allocation-free entry point (tfa_execute_noalloc): device memory of the loaded
// code object, one copy per GPU, held until the process ends.  Host code must never pass this
// name to a kernel (it is a host-side stand-in); it uses the per-device address from
// hipGetSymbolAddress (scratch_setup below).
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(TFA_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

bool is_pow2(int64_t n) { return n > 0 && (n & (n - 1)) == 0; }

// Largest power-of-two transform one workgroup keeps in LDS.
constexpr int64_t kMaxLdsN = 16384;
// Largest power-of-two transform of the two-pass four-step path (4096 x 4096).
constexpr int64_t kMaxFourStepN = int64_t(1) << 24;
// Smallest padded Bluestein length with the split three-pass path (m1 = m2 = 128), and the row
// count below which it replaces the fused kernel at m = 16384 (measured at 256 rows: fused 35.6
// us, split 57.3 us, so only a handful of rows, which leave most CUs idle, go split).
constexpr int64_t kMinBlueSplitM = 16384;
constexpr int64_t kBlueSplitRows = 64;

// exp(dir * 2*pi*i * num / den), num reduced mod den first; computed in fp64, rounded to fp32.
float2 unit_root(int64_t num, int64_t den, int dir) {
  num %= den;
  if (num < 0) num += den;
  const double a = 2.0 * M_PI * (double)num / (double)den;
  return make_float2((float)std::cos(a), (float)(dir * std::sin(a)));
}

// Twiddle table of the LDS Stockham transform of length n (layout of tfa::make_shape).
std::vector<float2> lds_table(int n, int dir, int e = 0) {
  const LdsShape s = tfa::make_shape(n, e ? e : tfa::lds_epth(n));
  std::vector<float2> t((size_t)s.twoff[s.npass] + 2, make_float2(1.0f, 0.0f));
  for (int p = 1; p < s.npass; ++p) {
    const int r = s.radix[p], ls = s.ls[p];
    for (int k = 0; k < ls; ++k)
      for (int q = 0; q < r; ++q) t[(size_t)s.twoff[p] + k * r + q] = unit_root((int64_t)q * k, (int64_t)ls * r, dir);
  }
  return t;
}

struct DevBuf {
  void* p = nullptr;
};

// Tables of the two-level fused Bluestein kernel at length m (tfa::blue_2l: m / b wavefronts of
// b = tfa::blue_2l_b(m) points per row, e = tfa::blue_2l_e(m) per lane): the wave transform's
// table (make_shape(b, e)), then from entry tfa::blue_2l_twoff(m) the rows W_m^(n_b w) (sign dir),
// w < m / b, n_b < b.
std::vector<float2> blue_2l_table(int m, int dir) {
  const int b = tfa::blue_2l_b(m), r = m / b, off = tfa::blue_2l_twoff(m);
  std::vector<float2> t = lds_table(b, dir, tfa::blue_2l_e(m));
  t.resize((size_t)off + (size_t)r * b, make_float2(1.0f, 0.0f));
  for (int w = 0; w < r; ++w)
    for (int nb = 0; nb < b; ++nb) t[(size_t)off + (size_t)w * b + nb] = unit_root((int64_t)nb * w, m, dir);
  return t;
}

// The filter spectrum in the two-level kernel's frequency order: entry t + (m / e) j of a row
// (wave w = t / 64, lane l = t % 64, element j) holds frequency w + (m / b) (l + 64 j).
std::vector<float2> blue_2l_permute(const std::vector<float2>& h) {
  const int mi = (int)h.size();
  const size_t m = h.size(), tt = m / tfa::blue_2l_e(mi), r = m / tfa::blue_2l_b(mi);
  std::vector<float2> out(m);
  for (size_t j = 0; j < m; ++j) {
    const size_t e = j / tt, w = (j % tt) >> 6, l = j & 63;
    out[j] = h[w + r * (l + 64 * e)];
  }
  return out;
}

// Power-of-two transform tables for one direction: LDS path (n <= kMaxLdsN) or four-step.
struct C2cTables {
  int64_t n = 0;
  int dir = -1;
  bool fourstep = false;
  float2* tw = nullptr;      // LDS path, batched kernel layout
  float2* tw_lds = nullptr;  // LDS path, strided / 2-D row kernel layout
  int n1 = 0, n2 = 0, lo_bits = 0;
  float2 *tw1 = nullptr, *tw2 = nullptr, *tw_lo = nullptr, *tw_hi = nullptr;
  int s_np = 0, s_len[3] = {0, 0, 0};  // strided multi-pass split of n >= 4096 (2 or 3 factors)
  float2* s_tw[3] = {nullptr, nullptr, nullptr};  // its per-factor tables (lds_epth layout)
};

}  // namespace

struct tfa_plan {
  tfa_plan_desc d{};
  int device = 0;
  int64_t m = 0;  // padded length (Bluestein: the reference's, trnfft/plan.py:42), else n
  int64_t mf = 0;  // Bluestein: internal length of the fused kernel (m, or a shorter mixed-radix length)
  C2cTables fwd, inv;  // C2C uses the one for its direction; Bluestein uses both (length m)
  bool blue_fused = false;  // Bluestein: fused one-launch kernel available (m <= 16384)
  bool blue_split = false;  // Bluestein: split three-pass path available (m >= 16384)
  int blue_m1 = 0, blue_m2 = 0, blue_lo_bits = 0;
  float2 *b_tw1f = nullptr, *b_tw1i = nullptr, *b_tw2f = nullptr, *b_tw2i = nullptr;
  float2 *b_lo = nullptr, *b_hi = nullptr, *b_hp = nullptr;
  float2* chirp = nullptr;
  float2* hs = nullptr;
  float2 *b_tw_sf = nullptr, *b_tw_si = nullptr;  // Bluestein m <= 4096: strided-axis kernel tables
  float2* b_hs_s = nullptr;  // Bluestein m <= 4096: strided-axis filter spectrum (length m, natural order; hs when mf == m and the fused kernel is one-level)
  float2* stft_hs_adj = nullptr;  // forward STFT, n_fft not a power of two: the adjoint chain's filter spectrum
  int blue_wrap = 0;         // Bluestein: 2n - 1 - mf when the fused length wraps the convolution
  C2cTables col;          // FFT2: LDS table for n2/8 (pass 2)
  float2* tw_h = nullptr;  // FFT2: W_{n2}^i, i < n2
  float2* tw_w_pair = nullptr;  // FFT2: row table in the paired-real-row layout
  float2 *tw_sw = nullptr, *tw_sh = nullptr;  // FFT2 small images: row / column tables
  float2* twr = nullptr;  // REAL: W_n^k, k < n/2
  float* w_re = nullptr;  // DFT-GEMM matrix
  float* w_im = nullptr;
  std::vector<void*> allocs;
  // set once the plan has been executed on a stream under graph capture: the captured kernels
  // hold raw pointers to these tables, so tfa_plan_destroy must not free them
  mutable std::atomic<bool> captured{false};

  ~tfa_plan() {
    for (void* p : allocs) (void)hipFree(p);
  }

  template <class T>
  int upload(const std::vector<T>& h, T** out) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, h.size() * sizeof(T) + 16);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(plan table)");
    allocs.push_back(p);
    e = hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy(plan table)");
    *out = static_cast<T*>(p);
    return TFA_OK;
  }

  int build_c2c(int64_t n, int dir, C2cTables* t) {
    t->n = n;
    t->dir = dir;
    if (n <= kMaxLdsN) {
      t->fourstep = false;
      // the batched kernel's layout (tfa::c2c_epth); the strided and 2-D row kernels use the
      // tfa::lds_epth layout, a second table only where the two differ
      int rc = upload(lds_table((int)n, dir, tfa::c2c_epth((int)n)), &t->tw);
      if (!rc && tfa::c2c_epth((int)n) != tfa::lds_epth((int)n)) rc = upload(lds_table((int)n, dir), &t->tw_lds);
      else t->tw_lds = t->tw;
      if (rc || n < tfa::kMinStridedMultiPassN) return rc;
      if ((rc = build_roots(n, dir, t))) return rc;
      return build_strided_split(n, dir, t);
    }
    if (n > kMaxFourStepN) return fail(TFA_ERR_UNSUPPORTED, "power-of-two length above 2^24 not supported");
    t->fourstep = true;
    int rc = build_split(n, dir, t);
    if (!rc) rc = build_strided_split(n, dir, t);
    return rc;
  }

  // W_n^j = W^lo * W^hi tables (j = hi << lo_bits | lo)
  int build_roots(int64_t n, int dir, C2cTables* t) {
    const int lg = tfa::ilog2(n);
    t->lo_bits = (lg + 1) / 2;
    std::vector<float2> lo((size_t)1 << t->lo_bits), hi((size_t)(n >> t->lo_bits));
    for (size_t j = 0; j < lo.size(); ++j) lo[j] = unit_root((int64_t)j, n, dir);
    for (size_t j = 0; j < hi.size(); ++j) hi[j] = unit_root((int64_t)j << t->lo_bits, n, dir);
    int rc = upload(lo, &t->tw_lo);
    return rc ? rc : upload(hi, &t->tw_hi);
  }

  // factors of a strided axis n >= 4096 (multi-pass strided path): two, n1 = 2^floor(lg/2) <= n2,
  // below 2^21; three of 128..256 from 2^21 (every pass with 64-column tiles)
  int build_strided_split(int64_t n, int dir, C2cTables* t) {
    const int lg = tfa::ilog2(n);
    int bits[3];
    if (lg >= tfa::kStridedThreePassLg) {
      t->s_np = 3;
      bits[0] = lg / 3;
      bits[1] = (lg - bits[0]) / 2;
      bits[2] = lg - bits[0] - bits[1];
    } else {
      t->s_np = 2;
      bits[0] = lg / 2;
      bits[1] = lg - bits[0];
    }
    for (int i = 0; i < t->s_np; ++i) {
      t->s_len[i] = 1 << bits[i];
      if (i > 0 && t->s_len[i] == t->s_len[i - 1]) {
        t->s_tw[i] = t->s_tw[i - 1];
        continue;
      }
      int rc = upload(lds_table(t->s_len[i], dir), &t->s_tw[i]);
      if (rc) return rc;
    }
    return TFA_OK;
  }

  // n = n1 * n2 (n1 = 2^floor(lg/2) <= n2, except 2^15 and 2^17, whose longer column transform
  // measured faster: 128 x 2^15 35.2 -> 32.8 us as 256 x 128, 32 x 2^17 32.7 -> 31.1 as
  // 512 x 256, while 2^19, 2^21 and 2^23 lost 3-10 % that way): LDS-FFT tables of both lengths
  // (tfa::fourstep_epth layout) and the two-level W_n^j tables of the twiddle between the passes
  int build_split(int64_t n, int dir, C2cTables* t) {
    const int lg = tfa::ilog2(n);
    t->n1 = 1 << ((lg == 15 || lg == 17) ? lg - lg / 2 : lg / 2);  // column transform length (strided)
    t->n2 = (int)(n / t->n1);                                      // row transform length (contiguous)
    t->lo_bits = (lg + 1) / 2;
    int rc;
    if ((rc = upload(lds_table(t->n1, dir, tfa::fourstep_epth(t->n1)), &t->tw1))) return rc;
    if ((rc = upload(lds_table(t->n2, dir, tfa::fourstep_epth(t->n2)), &t->tw2))) return rc;
    return build_roots(n, dir, t);
  }
};

namespace {

// Bluestein path choice: the fused kernel holds one row per workgroup, so with fewer than
// kBlueSplitRows rows it leaves most of the GPU idle and the split three-pass path (each row
// spread over many workgroups per pass) takes over; above 16384 only the split path exists.
// Internal length of the fused Bluestein kernel for n whose reference padded length is m (the
// smallest power of two >= 2n - 1).  Where 2n - 1 exceeds m/2 by at most kBlueWrapMax (n just
// above a power of two, e.g. C3b's 4099 = 4096 + 3), the kernel convolves circularly at m/2 and
// corrects the 2 * (2n - 1 - m/2) outputs the wrapped filter taps reach (exact, see the kernel):
// half the transform length (4099: 8192 points against 9216 or the reference's 16384).
// Otherwise the circular convolution needs L >= 2n - 1, and where m overshoots that by most, a
// mixed-radix length (3^2 * 2^10 = 9216 for 4096 < n <= 4608, against m = 16384) halves the
// transforms and the LDS (two workgroups per CU instead of one).
// Internal length of the fused Bluestein kernel: the wrapped power of two m/2 where at most
// kBlueWrapMax outputs need correcting, else the shortest measured-faster mixed-radix length that
// holds the 2n - 1 point convolution, else the reference's m.  12288 = 24 x 8^3 (four passes at 24
// elements per thread, 512 threads) for 4608 < n <= 6144: n = 5000 x 838 rows 102.5 -> 69.0 us,
// n = 6000 x 699 78.2 -> 53.3 against 16384 points.
int64_t blue_fused_length(int64_t n, int64_t m) {
  if (tfa::blue_wrap_ok((int)std::min<int64_t>(m / 2, 1 << 30)) && 2 * n - 1 - m / 2 <= tfa::kBlueWrapMax) return m / 2;
  for (int64_t c : {768, 1536, 3072, 9216, 12288})
    if (c >= 2 * n - 1 && c < m) return c;
  return m;
}

bool blue_use_split(const tfa_plan* p, int64_t batch) {
  if (!p->blue_fused) return true;
  // With few rows the fused kernel's shorter internal lengths still win where they are at most
  // 9216 points: n = 4099 at 9216 points, 1 row 12.7 vs 13.9 us for the split path at 16384, 16 rows
  // 13.8 vs 16.2, 63 rows 14.7 vs 23.0 (the wrapped 8192-point length: 10.8 us at 1 row).  The
  // 12288-point length (24 x 8^3, for 4608 < n <= 6144 against the reference's 16384) wins from
  // about 28 rows: n = 5000, 24 rows 17.6 vs 17.1 us split, 32 rows 17.7 vs 18.6, 838 rows 69 vs
  // 103 at 16384 points fused.
  if (p->mf == 12288) return p->blue_split && batch < 28;
  // The two-level kernel at 16384 points wins from about 36 rows at the reference's m (n = 7000:
  // 32 rows 19.1 vs 18.9 us split, 48 rows 19.2 vs 21.1) and at every batch where it wraps
  // (n = 8193: 8 rows 19.4 vs 20.6 us for the split path at 32768).
  if (p->mf == 16384) return p->blue_split && p->mf == p->m && batch < 36;
  return p->blue_split && batch < kBlueSplitRows && p->mf == p->m;
}

size_t c2c_workspace(const C2cTables& t, int64_t batch) {
  return t.fourstep ? (size_t)2 * sizeof(float) * (size_t)batch * (size_t)t.n : 0;
}

int run_c2c(const C2cTables& t, int64_t batch, const float* in_re, const float* in_im, float* out_re,
            float* out_im, void* ws, float scale, hipStream_t s) {
  hipError_t e;
  if (!t.fourstep) {
    tfa::C2cArgs a{in_re, in_im, out_re, out_im, t.tw, batch, scale, t.dir, s};
    e = tfa::launch_c2c_lds((int)t.n, a);
  } else {
    if (!ws) return fail(TFA_ERR_INVALID, "four-step transform needs a workspace");
    float* t_re = static_cast<float*>(ws);
    float* t_im = t_re + (size_t)batch * (size_t)t.n;
    if (t.s_np == 3 && tfa::ilog2(t.n) >= tfa::kContigThreePassLg) {
      // three passes over factors <= 256 (64-column tiles) instead of the two-pass four-step,
      // whose 2048- and 4096-point passes have 16- and 8-column tiles
      tfa::StridedFourStepArgs a{in_re, in_im, t_re, t_im, out_re, out_im, t.s_np, {t.s_len[0], t.s_len[1], t.s_len[2]},
                                 {t.s_tw[0], t.s_tw[1], t.s_tw[2]}, t.tw_lo, t.tw_hi, t.lo_bits, batch, 1, scale, t.dir, s};
      e = tfa::launch_strided_fourstep(a);
    } else {
      tfa::FourStepArgs a{in_re, in_im, t_re, t_im, out_re, out_im, t.tw1, t.tw2, t.tw_lo, t.tw_hi,
                          t.n1, t.n2, t.lo_bits, batch, scale, t.dir, s};
      e = tfa::launch_fourstep(a);
    }
  }
  return e == hipSuccess ? TFA_OK : hip_fail(e, "c2c launch");
}

// Host fp64 radix-2 FFT (forward, in place) used only to build the Bluestein filter spectrum.
void host_fft(std::vector<std::complex<double>>& a);

// Host fp64 forward DFT of a power-of-two length, or of 3^a * 2^b (one radix-3 split per factor 3
// down to the radix-2 FFT); builds the filter spectrum of the mixed-radix fused lengths.
void host_dft(std::vector<std::complex<double>>& a) {
  const size_t n = a.size();
  if (n % 3 != 0) {
    host_fft(a);
    return;
  }
  const size_t q = n / 3;
  std::vector<std::complex<double>> s[3];
  for (int r = 0; r < 3; ++r) {
    s[r].resize(q);
    for (size_t j = 0; j < q; ++j) s[r][j] = a[3 * j + r];
    host_dft(s[r]);
  }
  for (size_t k = 0; k < n; ++k) {
    std::complex<double> acc = s[0][k % q];
    for (int r = 1; r < 3; ++r) {
      const double ang = -2.0 * M_PI * (double)((r * k) % n) / (double)n;
      acc += s[r][k % q] * std::complex<double>(std::cos(ang), std::sin(ang));
    }
    a[k] = acc;
  }
}

void host_fft(std::vector<std::complex<double>>& a) {
  const size_t n = a.size();
  for (size_t i = 1, j = 0; i < n; ++i) {
    size_t bit = n >> 1;
    for (; j & bit; bit >>= 1) j ^= bit;
    j ^= bit;
    if (i < j) std::swap(a[i], a[j]);
  }
  for (size_t len = 2; len <= n; len <<= 1) {
    for (size_t k = 0; k < len / 2; ++k) {
      const double ang = -2.0 * M_PI * (double)k / (double)len;
      const std::complex<double> w(std::cos(ang), std::sin(ang));
      for (size_t i = k; i < n; i += len) {
        const std::complex<double> u = a[i], v = a[i + len / 2] * w;
        a[i] = u + v;
        a[i + len / 2] = u - v;
      }
    }
  }
}

// The reference's chirp, trnfft/fft_core.py:1316-1320: angle = sign * pi * k * k / n evaluated
// in fp32 exactly as torch does it (fp32(sign*pi) * k, * k, true division by n, each rounded
// to fp32), then cos/sin of that fp32 angle.  Reproducing the fp32 angle is required for parity:
// its rounding moves the reference's result ~1e-4 (n=1000) from the exact DFT.
std::vector<float2> reference_chirp(int64_t n, int sign) {
  std::vector<float2> c((size_t)n);
  volatile float spi = (float)(sign * M_PI);
  const float fn = (float)n;
  for (int64_t k = 0; k < n; ++k) {
    const float kf = (float)k;
    volatile float a1 = spi * kf;
    volatile float a2 = a1 * kf;
    volatile float a3 = a2 / fn;
    const double a = (double)a3;
    c[(size_t)k] = make_float2((float)std::cos(a), (float)std::sin(a));
  }
  return c;
}

// Bluestein filter spectrum: h = conj(chirp) circularly wrapped (trnfft/fft_core.py:1337-1345)
// to the circular convolution length L; H = FFT_L(h) / L.  Any L >= 2n - 1 gives the same
// convolution, so the fused kernel may use a shorter mixed-radix length than the reference's m;
// below 2n - 1 the taps i and L - i (i > L - n) share a slot and are summed (the wrapped fused
// kernel corrects the outputs they reach).  kmax < n keeps only the taps -(n-1) .. kmax-1, all
// that outputs k < kmax read: then any L >= n + kmax - 1 gives their values without wrap-around.
std::vector<float2> blue_taps_spectrum(const std::vector<float2>& chirp, int64_t L, int64_t pos, int64_t neg,
                                       bool conj_taps) {
  std::vector<std::complex<double>> h((size_t)L, {0.0, 0.0});
  for (int64_t i = 0; i < (int64_t)chirp.size(); ++i) {
    const std::complex<double> hc(chirp[(size_t)i].x, conj_taps ? -(double)chirp[(size_t)i].y : (double)chirp[(size_t)i].y);
    if (i < pos) h[(size_t)i] += hc;
    if (i > 0 && i < neg) h[(size_t)(L - i)] += hc;
  }
  host_dft(h);
  std::vector<float2> hs((size_t)L);
  for (int64_t i = 0; i < L; ++i)
    hs[(size_t)i] = make_float2((float)(h[(size_t)i].real() / (double)L), (float)(h[(size_t)i].imag() / (double)L));
  return hs;
}

std::vector<float2> blue_filter_spectrum(const std::vector<float2>& chirp, int64_t L, int64_t kmax = -1) {
  const int64_t n = (int64_t)chirp.size();
  return blue_taps_spectrum(chirp, L, kmax < 0 ? n : kmax, n, true);
}

// Filter spectrum of the adjoint of the truncated chain (outputs k < kmax): the adjoint maps
// u_k (k < kmax) to v_j = sum_k u_k chirp[|j - k|] (j < n), a convolution with the taps
// -(kmax-1) .. n-1 of chirp[|s|] (not conjugated), also / L.
std::vector<float2> blue_adjoint_spectrum(const std::vector<float2>& chirp, int64_t L, int64_t kmax) {
  return blue_taps_spectrum(chirp, L, (int64_t)chirp.size(), kmax, false);
}

std::mutex g_retained_mu;

// plans destroyed after use under graph capture (never freed; see tfa_plan_destroy)
std::vector<tfa_plan*>& retained_plans() {
  static std::vector<tfa_plan*>* v = new std::vector<tfa_plan*>();
  return *v;
}

// Marks the plan as referenced by a captured graph when `stream` is capturing.  The null stream
// never captures (and querying it while another stream captures in global mode is an error).
void note_capture(const tfa_plan* plan, tfa_stream stream) {
  if (!stream || plan->captured.load(std::memory_order_relaxed)) return;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &st) != hipSuccess) {
    (void)hipGetLastError();  // leave no error behind for the launch check that follows
    return;
  }
  if (st != hipStreamCaptureStatusNone) plan->captured.store(true, std::memory_order_release);
}

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;  // held across a noalloc call's wait, launch and record (per process)
void* g_scratch_ptr[kMaxScratchDevices] = {};
hipEvent_t g_scratch_done[kMaxScratchDevices] = {};  // recorded after each eager noalloc call
bool g_scratch_used[kMaxScratchDevices] = {};

// Set-up of the noalloc scratch on `dev`, which must be the current device (first call on each
// device, g_scratch_mu held): the device address of `scratch` and the event that orders the
// calls sharing it.
int scratch_setup(int dev) {
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(TFA_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags(noalloc order)");
    g_scratch_done[dev] = ev;
    g_scratch_ptr[dev] = p;
  }
  return TFA_OK;
}

}  // namespace

extern "C" {

int32_t tfa_abi_version(void) { return (1 << 16) | 2; }

const char* tfa_last_error(void) { return g_last_error.c_str(); }

int tfa_plan_create(tfa_plan** out, const tfa_plan_desc* desc) {
  if (!out || !desc) return fail(TFA_ERR_INVALID, "null argument");
  *out = nullptr;
  const int64_t n = desc->n;
  if (n < 1) return fail(TFA_ERR_INVALID, "transform length must be >= 1");
  tfa_plan* p = new (std::nothrow) tfa_plan();
  if (!p) return fail(TFA_ERR_INVALID, "out of host memory");
  p->d = *desc;
  p->m = n;
  hipError_t he = hipGetDevice(&p->device);
  if (he != hipSuccess) {
    delete p;
    return hip_fail(he, "hipGetDevice");
  }
  const int dir = desc->inverse ? 1 : -1;
  int rc = TFA_OK;
  switch (desc->kind) {
    case TFA_KIND_C2C:
      if (!is_pow2(n)) {
        rc = fail(TFA_ERR_INVALID, "TFA_KIND_C2C needs a power-of-two length");
        break;
      }
      rc = p->build_c2c(n, dir, dir < 0 ? &p->fwd : &p->inv);
      break;
    case TFA_KIND_BLUESTEIN: {
      if (n < 2) {
        rc = fail(TFA_ERR_INVALID, "Bluestein needs n >= 2");
        break;
      }
      // trnfft/plan.py:42: m = 1 << (2n-2).bit_length()
      int64_t v = 2 * n - 2, bits = 0;
      while (v) { ++bits; v >>= 1; }
      const int64_t m = int64_t(1) << bits;
      p->m = m;
      if (m > kMaxFourStepN) {
        rc = fail(TFA_ERR_UNSUPPORTED, "Bluestein padded length above 2^24 not supported");
        break;
      }
      p->mf = blue_fused_length(n, m);
      p->blue_fused = p->mf <= kMaxLdsN;
      p->blue_split = m >= kMinBlueSplitM;
      if (!p->blue_fused) p->mf = 0;
      p->blue_wrap = p->blue_fused && p->mf < 2 * n - 1 ? (int)(2 * n - 1 - p->mf) : 0;
      if (p->blue_fused) {
        // the fused kernel's own launch shape (tfa::blue_epth) fixes its table layout
        const int mf = (int)p->mf;
        p->fwd.n = p->inv.n = mf;
        p->fwd.dir = -1;
        p->inv.dir = 1;
        if (tfa::blue_2l(mf)) {  // the two-level kernel's tables (tfa::bluestein_2l_kernel)
          if ((rc = p->upload(blue_2l_table(mf, -1), &p->fwd.tw))) break;
          if ((rc = p->upload(blue_2l_table(mf, 1), &p->inv.tw))) break;
        } else {
          if ((rc = p->upload(lds_table(mf, -1, tfa::blue_epth(mf)), &p->fwd.tw))) break;
          if ((rc = p->upload(lds_table(mf, 1, tfa::blue_epth(mf)), &p->inv.tw))) break;
        }
        if (m <= tfa::kMaxStridedBlueM) {  // the strided-axis kernel's layout (tfa::lds_epth)
          if (p->mf == m && !tfa::blue_2l((int)m) && tfa::blue_epth((int)m) == tfa::lds_epth((int)m)) {
            p->b_tw_sf = p->fwd.tw;
            p->b_tw_si = p->inv.tw;
          } else {
            if ((rc = p->upload(lds_table((int)m, -1), &p->b_tw_sf))) break;
            if ((rc = p->upload(lds_table((int)m, 1), &p->b_tw_si))) break;
          }
        }
      }
      const std::vector<float2> chirp = reference_chirp(n, dir);
      auto filter_spectrum = [&](int64_t L) { return blue_filter_spectrum(chirp, L); };
      const std::vector<float2> hs = filter_spectrum(m);
      if ((rc = p->upload(chirp, &p->chirp))) break;
      if (p->blue_fused && tfa::blue_2l((int)p->mf)) {
        if ((rc = p->upload(blue_2l_permute(filter_spectrum(p->mf)), &p->hs))) break;
      } else if ((rc = p->upload(p->blue_fused && p->mf != m ? filter_spectrum(p->mf) : hs, &p->hs))) {
        break;
      }
      if (m <= tfa::kMaxStridedBlueM) {
        // (the strided-axis kernel reads H/m in natural order; the two-level fused kernel's copy is
        // permuted)
        if (p->mf == m && !tfa::blue_2l((int)p->mf)) p->b_hs_s = p->hs;
        else if ((rc = p->upload(hs, &p->b_hs_s))) break;
      }
      if (p->blue_split) {
        // m = m1 * m2 (m1 = 2^floor(log2 m / 2)); tables of the three passes, H/m permuted to
        // the transposed spectrum order hp[k1*m2 + k2] = H[k1 + m1*k2] / m
        const int lg = tfa::ilog2((int)m);
        p->blue_m1 = 1 << (lg / 2);
        p->blue_m2 = (int)(m / p->blue_m1);
        p->blue_lo_bits = (lg + 1) / 2;
        const int m1 = p->blue_m1, m2 = p->blue_m2;
        if ((rc = p->upload(lds_table(m1, -1, tfa::blue_col_epth(m1)), &p->b_tw1f))) break;
        if ((rc = p->upload(lds_table(m1, 1, tfa::blue_col_epth(m1)), &p->b_tw1i))) break;
        if ((rc = p->upload(lds_table(m2, -1, tfa::c2c_epth(m2)), &p->b_tw2f))) break;
        if ((rc = p->upload(lds_table(m2, 1, tfa::c2c_epth(m2)), &p->b_tw2i))) break;
        std::vector<float2> lo((size_t)1 << p->blue_lo_bits), hi((size_t)(m >> p->blue_lo_bits));
        for (size_t j = 0; j < lo.size(); ++j) lo[j] = unit_root((int64_t)j, m, -1);
        for (size_t j = 0; j < hi.size(); ++j) hi[j] = unit_root((int64_t)j << p->blue_lo_bits, m, -1);
        if ((rc = p->upload(lo, &p->b_lo))) break;
        if ((rc = p->upload(hi, &p->b_hi))) break;
        std::vector<float2> hp((size_t)m);
        for (int k1 = 0; k1 < m1; ++k1)
          for (int k2 = 0; k2 < m2; ++k2) hp[(size_t)k1 * m2 + k2] = hs[(size_t)k1 + (size_t)m1 * k2];
        rc = p->upload(hp, &p->b_hp);
      }
      break;
    }
    case TFA_KIND_STFT:
      if (desc->hop < 1) {
        rc = fail(TFA_ERR_INVALID, "hop_length must be >= 1");
        break;
      }
      if (!is_pow2(n)) {
        // forward STFT with one Bluestein transform per frame (the reference's chain,
        // trnfft/fft_core.py:1285-1376): chirp, the filter spectrum H/m of the taps that the kept
        // bins read, and the two m-point LDS tables; m is the shortest power of two or 3 * 2^k
        // with n + n_bins - 1 <= m (the reference pads to the power of two >= 2n - 1)
        // (inverse: every sample of a frame is kept, so m >= 2n - 1, with the chirp of sign +1,
        // trnfft/api.py:412-417 -> fft_core.py:1285-1376)
        const int64_t bins = (desc->flags & TFA_STFT_ONESIDED) ? n / 2 + 1 : n;
        const int64_t conv = desc->inverse ? 2 * n - 1 : n + bins - 1;
        int64_t m = 0;
        for (int64_t c = tfa::kStftBlueMinM; c <= tfa::kStftBlueMaxM && !m; ++c)
          if (tfa::stft_blue_len_ok(c) && conv <= c && n <= tfa::stft_blue_nmax((int)c)) m = c;
        if (n < 9 || m == 0) {
          rc = fail(TFA_ERR_UNSUPPORTED, desc->inverse
                        ? "fused inverse STFT: n_fft that is not a power of two must lie in 9..2048"
                        : "fused STFT: n_fft that is not a power of two must lie in 9..2731 onesided or 9..2048 two-sided");
          break;
        }
        if (desc->inverse) {
          if (!(desc->flags & TFA_STFT_ONESIDED)) {
            rc = fail(TFA_ERR_UNSUPPORTED, "fused inverse STFT at an n_fft that is not a power of two takes onesided spectra");
            break;
          }
          // a halo of more than half the tile recomputes more frames than it owns: the composed
          // path is faster there
          if (2 * ((n - 1) / desc->hop) > tfa::istft_blue_frames((int)m)) {
            rc = fail(TFA_ERR_UNSUPPORTED, "hop_length too small for the fused inverse STFT tile");
            break;
          }
        }
        const int e = desc->inverse ? tfa::istft_blue_epth((int)m) : tfa::stft_blue_epth((int)m);
        p->m = p->mf = m;
        p->fwd.n = p->inv.n = m;
        p->fwd.dir = -1;
        p->inv.dir = 1;
        const std::vector<float2> chirp = reference_chirp(n, desc->inverse ? 1 : -1);
        if ((rc = p->upload(lds_table((int)m, -1, e), &p->fwd.tw))) break;
        if ((rc = p->upload(lds_table((int)m, 1, e), &p->inv.tw))) break;
        if ((rc = p->upload(chirp, &p->chirp))) break;
        if ((rc = p->upload(blue_filter_spectrum(chirp, m, desc->inverse ? n : bins), &p->hs))) break;
        // the forward plan also serves the signal gradient (tfa_stft_backward_execute), onesided
        if (!desc->inverse && (desc->flags & TFA_STFT_ONESIDED))
          rc = p->upload(blue_adjoint_spectrum(chirp, m, bins), &p->stft_hs_adj);
        break;
      }
      if (n < 16 || n > 4096) {
        rc = fail(TFA_ERR_UNSUPPORTED, "fused STFT needs a power-of-two n_fft in [16, 4096]");
        break;
      }
      if (desc->inverse) {
        // inverse STFT (onesided spectra, or two-sided ones: the real part of each frame's inverse
        // transform): inverse table in the pair-transform layout of the istft kernel
        if ((n - 1) / desc->hop >= tfa::istft_frames_per_tile((int)n, !(desc->flags & TFA_STFT_ONESIDED))) {
          rc = fail(TFA_ERR_UNSUPPORTED, "hop_length too small for the fused inverse STFT tile");
          break;
        }
        p->inv.n = n;
        p->inv.dir = 1;
        rc = p->upload(lds_table((int)n, 1, tfa::istft_epth((int)n)), &p->inv.tw);
        break;
      }
      p->fwd.n = n;
      p->fwd.dir = -1;
      if ((rc = p->upload(lds_table((int)n, -1, tfa::stft_epth((int)n)), &p->fwd.tw))) break;
      // the signal gradient (tfa_stft_backward_execute) runs on the inverse kernel's layout
      p->inv.n = n;
      p->inv.dir = 1;
      rc = p->upload(lds_table((int)n, 1, tfa::istft_epth((int)n)), &p->inv.tw);
      break;
    case TFA_KIND_FFT2: {
      const int64_t h = desc->n2;
      if (tfa::fft2_small_ok(h, n)) {  // whole images in LDS: single pass
        const int e = tfa::fft2_small_epth((int)h, (int)n);
        p->fwd.n = n;
        p->fwd.dir = dir;
        if ((rc = p->upload(lds_table((int)n, dir, e), &p->tw_sw))) break;
        rc = p->upload(lds_table((int)h, dir, e), &p->tw_sh);
        break;
      }
      if (!is_pow2(n) || n < 16 || n > 4096 || !is_pow2(h) || h < 16 || h > 4096) {
        rc = fail(TFA_ERR_UNSUPPORTED,
                  "FFT2 plans need power-of-two 16 <= n <= 4096 and 16 <= n2 <= 4096, or n * n2 <= 16384 "
                  "with both axes >= 4 (and >= 8 / 16 at n * n2 = 8192 / 16384)");
        break;
      }
      if ((rc = p->build_c2c(n, dir, &p->fwd))) break;
      if ((rc = p->upload(lds_table((int)n, dir, tfa::fft2_pair_epth((int)n)), &p->tw_w_pair))) break;
      p->col.n = h / 8;
      p->col.dir = dir;
      if ((rc = p->upload(lds_table((int)(h / 8), dir, tfa::fft2_col_epth((int)(h / 8))), &p->col.tw))) break;
      std::vector<float2> th((size_t)h);
      for (int64_t i = 0; i < h; ++i) th[(size_t)i] = unit_root(i, h, dir);
      rc = p->upload(th, &p->tw_h);
      break;
    }
    case TFA_KIND_REAL: {
      if (!is_pow2(n) || n < 4 || n > 2 * kMaxLdsN) {
        rc = fail(TFA_ERR_UNSUPPORTED, "real-input plans need a power-of-two n in [4, 32768]");
        break;
      }
      // half-length transform table for the real kernels' own elements-per-thread choice
      C2cTables* t = dir < 0 ? &p->fwd : &p->inv;
      t->n = n / 2;
      t->dir = dir;
      if ((rc = p->upload(lds_table((int)(n / 2), dir, tfa::real_epth((int)(n / 2), dir > 0)), &t->tw))) break;
      std::vector<float2> tr((size_t)(n / 2));
      for (int64_t k = 0; k < n / 2; ++k) tr[(size_t)k] = unit_root(k, n, -1);
      rc = p->upload(tr, &p->twr);
      break;
    }
    case TFA_KIND_DFT_GEMM: {
      if (n > 4096) {
        rc = fail(TFA_ERR_UNSUPPORTED, "DFT-GEMM plans are limited to n <= 4096");
        break;
      }
      // exact DFT matrix: phase (k*j mod n) in integers, angle in fp64 (the reference builds
      // it from an fp32 angle, trnfft/fft_core.py:239-243, which costs ~2e-5 relative at n=256)
      std::vector<float> wr((size_t)(n * n)), wi((size_t)(n * n));
      for (int64_t k = 0; k < n; ++k)
        for (int64_t j = 0; j < n; ++j) {
          const float2 w = unit_root((k * j) % n, n, dir);
          wr[(size_t)(k * n + j)] = w.x;
          wi[(size_t)(k * n + j)] = w.y;
        }
      if ((rc = p->upload(wr, &p->w_re))) break;
      rc = p->upload(wi, &p->w_im);
      break;
    }
    default:
      rc = fail(TFA_ERR_INVALID, "unknown plan kind");
  }
  if (rc != TFA_OK) {
    delete p;
    return rc;
  }
  *out = p;
  return TFA_OK;
}

void tfa_plan_destroy(tfa_plan* plan) {
  if (!plan) return;
  if (plan->captured.load(std::memory_order_acquire)) {
    // a captured graph may still be replayed: keep the tables for the life of the process
    std::lock_guard<std::mutex> g(g_retained_mu);
    retained_plans().push_back(plan);
    return;
  }
  delete plan;
}

int64_t tfa_plan_padded_n(const tfa_plan* plan) { return plan ? plan->m : 0; }

int tfa_plan_workspace_size(const tfa_plan* plan, int64_t batch, size_t* bytes) {
  if (!plan || !bytes || batch < 0) return fail(TFA_ERR_INVALID, "bad argument");
  *bytes = 0;
  switch (plan->d.kind) {
    case TFA_KIND_C2C:
      *bytes = c2c_workspace(plan->d.inverse ? plan->inv : plan->fwd, batch);
      break;
    case TFA_KIND_BLUESTEIN:
      if (blue_use_split(plan, batch)) *bytes = (size_t)2 * sizeof(float) * (size_t)batch * (size_t)plan->m;
      break;
    default:
      break;
  }
  return TFA_OK;
}

int tfa_execute(const tfa_plan* plan, int64_t batch, const float* in_re, const float* in_im,
                float* out_re, float* out_im, void* workspace, tfa_stream stream) {
  if (!plan) return fail(TFA_ERR_INVALID, "null plan");
  if (batch < 0) return fail(TFA_ERR_INVALID, "negative batch");
  if (batch == 0) return TFA_OK;
  const bool c2r = plan->d.kind == TFA_KIND_REAL && plan->d.inverse;
  if (!in_re || !out_re || (!out_im && !c2r)) return fail(TFA_ERR_INVALID, "null data pointer");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != plan->device)
    return fail(TFA_ERR_INVALID, "plan was created on another device than the current one");
  note_capture(plan, stream);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n = plan->d.n;
  const float scale = plan->d.inverse ? (float)(1.0 / (double)n) : 1.0f;
  switch (plan->d.kind) {
    case TFA_KIND_C2C:
      return run_c2c(plan->d.inverse ? plan->inv : plan->fwd, batch, in_re, in_im, out_re, out_im,
                     workspace, scale, s);
    case TFA_KIND_BLUESTEIN: {
      tfa::BluesteinArgs a{in_re, in_im, out_re, out_im, plan->chirp, plan->hs, plan->fwd.tw,
                           plan->inv.tw, (int)n, (int)plan->mf, batch, scale, s, plan->blue_wrap};
      hipError_t e;
      if (!blue_use_split(plan, batch)) {
        e = tfa::launch_bluestein_fused((int)plan->mf, a);
        return e == hipSuccess ? TFA_OK : hip_fail(e, "bluestein launch");
      }
      if (!workspace) return fail(TFA_ERR_INVALID, "split Bluestein needs a workspace (tfa_plan_workspace_size)");
      float* y_re = static_cast<float*>(workspace);
      float* y_im = y_re + (size_t)batch * (size_t)plan->m;
      tfa::BlueSplitArgs sa{in_re, in_im, out_re, out_im, y_re, y_im, plan->chirp, plan->b_hp, plan->b_tw1f,
                            plan->b_tw1i, plan->b_tw2f, plan->b_tw2i, plan->b_lo, plan->b_hi, plan->blue_lo_bits,
                            (int)n, batch, scale, s};
      e = tfa::launch_bluestein_split(plan->blue_m1, plan->blue_m2, sa);
      return e == hipSuccess ? TFA_OK : hip_fail(e, "bluestein split launch");
    }
    case TFA_KIND_FFT2: {
      if (in_re == out_re || (in_im && in_im == out_im)) return fail(TFA_ERR_INVALID, "FFT2 output must not alias the input");
      const int64_t h = plan->d.n2;
      const float s2 = plan->d.inverse ? (float)(1.0 / ((double)n * (double)h)) : 1.0f;
      tfa::Fft2Args f{in_re, in_im, out_re, out_im, plan->fwd.tw_lds, plan->tw_w_pair, plan->col.tw, plan->tw_h,
                      plan->tw_sw, plan->tw_sh, batch, h, n, s2, plan->fwd.dir, s};
      hipError_t e = tfa::launch_fft2(f);
      return e == hipSuccess ? TFA_OK : hip_fail(e, "fft2 launch");
    }
    case TFA_KIND_REAL: {
      const float* rows = c2r ? out_re : in_re;
      if (reinterpret_cast<uintptr_t>(rows) % 8 != 0) return fail(TFA_ERR_INVALID, "real rows must be 8-byte aligned");
      if (c2r ? !in_im : in_im != nullptr)
        return fail(TFA_ERR_INVALID, c2r ? "c2r needs both input planes" : "r2c takes real input (in_im must be NULL)");
      if (in_re == out_re || (c2r && in_im == out_re) || (!c2r && in_re == out_im))
        return fail(TFA_ERR_INVALID, "real transforms are out-of-place only");
      const C2cTables& t = c2r ? plan->inv : plan->fwd;
      tfa::RealArgs a{in_re, in_im, out_re, out_im, t.tw, plan->twr, batch, scale, c2r, s};
      hipError_t e = tfa::launch_real((int)n, a);
      return e == hipSuccess ? TFA_OK : hip_fail(e, "real transform launch");
    }
    case TFA_KIND_DFT_GEMM: {
      if (!in_im) return fail(TFA_ERR_INVALID, "DFT-GEMM needs both input planes");
      // X = x @ W (W symmetric, so x @ W^T), scaled 1/n when inverse
      tfa::GemmArgs g{batch, n, n, in_re, in_im, n, TFA_OP_N, plan->w_re, plan->w_im, n, TFA_OP_T,
                      nullptr, nullptr, out_re, out_im, n, scale, s};
      hipError_t e = tfa::launch_cgemm(g);
      return e == hipSuccess ? TFA_OK : hip_fail(e, "dft-gemm launch");
    }
    default:
      return fail(TFA_ERR_UNSUPPORTED, "plan kind not executable with tfa_execute");
  }
}

namespace {

// power-of-two C2C axis longer than the single-pass strided kernel: two strided passes
bool strided_fourstep(const tfa_plan* plan, int64_t stride) {
  if (plan->d.kind != TFA_KIND_C2C || plan->d.n < tfa::kMinStridedMultiPassN) return false;
  const C2cTables& t = plan->d.inverse ? plan->inv : plan->fwd;
  return stride >= tfa::strided_fs_min_stride(t.s_np, plan->d.n);
}

}  // namespace

int tfa_strided_workspace_size(const tfa_plan* plan, int64_t outer, int64_t stride, size_t* bytes) {
  if (!plan || !bytes) return fail(TFA_ERR_INVALID, "null argument");
  if (outer < 0 || stride < 1) return fail(TFA_ERR_INVALID, "bad outer/stride");
  *bytes = strided_fourstep(plan, stride) ? (size_t)2 * sizeof(float) * (size_t)outer * (size_t)plan->d.n * (size_t)stride : 0;
  return TFA_OK;
}

int tfa_execute_noalloc(const tfa_plan* plan, int64_t batch, const float* in_re, const float* in_im,
                        float* out_re, float* out_im, tfa_stream stream) {
  if (!plan) return fail(TFA_ERR_INVALID, "null plan");
  if (batch < 0) return fail(TFA_ERR_INVALID, "negative batch");
  size_t need = 0;
  int rc = tfa_plan_workspace_size(plan, batch, &need);
  if (rc) return rc;
  if (need > kNoAllocScratchBytes)
    return fail(TFA_ERR_INVALID, "tfa_execute_noalloc: this transform needs " + std::to_string(need) +
                                     " bytes of scratch, above the static scratch of " +
                                     std::to_string(kNoAllocScratchBytes) + " bytes (use tfa_execute with a workspace)");
  if (need == 0) return tfa_execute(plan, batch, in_re, in_im, out_re, out_im, nullptr, stream);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != plan->device)
    return fail(TFA_ERR_INVALID, "plan was created on another device than the current one");
  if (dev < 0 || dev >= kMaxScratchDevices) return fail(TFA_ERR_UNSUPPORTED, "device index beyond the scratch table");
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if ((rc = scratch_setup(dev))) return rc;
  // every call on this GPU shares the scratch: an eager call waits on the device for the previous
  // eager call's kernels (on whatever stream) before its own use it.  Calls captured into a graph
  // are not ordered (a captured wait on an event recorded outside the capture is not allowed):
  // replays that overlap other noalloc calls on this GPU race.
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    st = hipStreamCaptureStatusNone;
  }
  const bool eager = st == hipStreamCaptureStatusNone;
  if (eager && g_scratch_used[dev]) {
    const hipError_t e = hipStreamWaitEvent(s, g_scratch_done[dev], 0);
    if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent(noalloc order)");
  }
  // the same kernels as tfa_execute; every kernel writes the scratch it later reads, so nothing
  // needs clearing between calls
  rc = tfa_execute(plan, batch, in_re, in_im, out_re, out_im, g_scratch_ptr[dev], stream);
  if (rc == TFA_OK && eager) {
    const hipError_t e = hipEventRecord(g_scratch_done[dev], s);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord(noalloc order)");
    g_scratch_used[dev] = true;
  }
  return rc;
}

int tfa_execute_strided_ws(const tfa_plan* plan, int64_t outer, int64_t stride, const float* in_re,
                           const float* in_im, float* out_re, float* out_im, void* workspace, tfa_stream stream) {
  if (!plan) return fail(TFA_ERR_INVALID, "null plan");
  if (!strided_fourstep(plan, stride))
    return tfa_execute_strided(plan, outer, stride, in_re, in_im, out_re, out_im, stream);
  if (outer < 0) return fail(TFA_ERR_INVALID, "bad outer/stride");
  if (outer == 0) return TFA_OK;
  if (!in_re || !out_re || !out_im) return fail(TFA_ERR_INVALID, "null data pointer");
  if (!workspace) return fail(TFA_ERR_INVALID, "strided four-step transform needs a workspace");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != plan->device)
    return fail(TFA_ERR_INVALID, "plan was created on another device than the current one");
  note_capture(plan, stream);
  const C2cTables& t = plan->d.inverse ? plan->inv : plan->fwd;
  const size_t plane = (size_t)outer * (size_t)plan->d.n * (size_t)stride;
  float* t_re = static_cast<float*>(workspace);
  const float scale = plan->d.inverse ? (float)(1.0 / (double)plan->d.n) : 1.0f;
  tfa::StridedFourStepArgs a{in_re, in_im, t_re, t_re + plane, out_re, out_im, t.s_np, {t.s_len[0], t.s_len[1], t.s_len[2]},
                             {t.s_tw[0], t.s_tw[1], t.s_tw[2]}, t.tw_lo, t.tw_hi, t.lo_bits, outer, stride, scale, t.dir,
                             static_cast<hipStream_t>(stream)};
  hipError_t e = tfa::launch_strided_fourstep(a);
  if (e == hipErrorInvalidValue) return fail(TFA_ERR_UNSUPPORTED, "strided four-step: shape beyond the launch grid");
  return e == hipSuccess ? TFA_OK : hip_fail(e, "strided four-step launch");
}

int tfa_execute_strided(const tfa_plan* plan, int64_t outer, int64_t stride, const float* in_re,
                        const float* in_im, float* out_re, float* out_im, tfa_stream stream) {
  if (!plan) return fail(TFA_ERR_INVALID, "null plan");
  if (outer < 0 || stride < 1) return fail(TFA_ERR_INVALID, "bad outer/stride");
  const bool blue = plan->d.kind == TFA_KIND_BLUESTEIN && plan->m <= tfa::kMaxStridedBlueM;
  // the workspace query reports 0 bytes for outer = 0, which sends callers here: an empty call
  // is a no-op for every shape the workspace entry point runs too
  if (outer == 0 && strided_fourstep(plan, stride)) return TFA_OK;
  if (!blue && (plan->d.kind != TFA_KIND_C2C || plan->d.n > tfa::kMaxStridedN || plan->d.n < 2))
    return fail(TFA_ERR_UNSUPPORTED,
                "strided transforms need a power-of-two C2C plan with 2 <= n <= 4096 or a Bluestein plan with n <= 2048 "
                "(longer power-of-two axes with stride >= 4, >= 8 from 2^21: tfa_execute_strided_ws)");
  if (outer == 0) return TFA_OK;
  if (!in_re || !out_re || !out_im) return fail(TFA_ERR_INVALID, "null data pointer");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != plan->device)
    return fail(TFA_ERR_INVALID, "plan was created on another device than the current one");
  note_capture(plan, stream);
  if (blue) {
    const float bscale = plan->d.inverse ? (float)(1.0 / (double)plan->d.n) : 1.0f;
    tfa::StridedBlueArgs ba{in_re, in_im, out_re, out_im, plan->chirp, plan->b_hs_s, plan->b_tw_sf, plan->b_tw_si,
                            outer, stride, (int)plan->d.n, bscale, static_cast<hipStream_t>(stream)};
    hipError_t be = tfa::launch_strided_bluestein((int)plan->m, ba);
    return be == hipSuccess ? TFA_OK : hip_fail(be, "strided Bluestein launch");
  }
  const C2cTables& t = plan->d.inverse ? plan->inv : plan->fwd;
  const float scale = plan->d.inverse ? (float)(1.0 / (double)plan->d.n) : 1.0f;
  tfa::StridedArgs a{in_re, in_im, out_re, out_im, t.tw_lds, outer, stride, scale, t.dir,
                     static_cast<hipStream_t>(stream)};
  hipError_t e = tfa::launch_strided((int)plan->d.n, a);
  return e == hipSuccess ? TFA_OK : hip_fail(e, "strided launch");
}

int tfa_stft_frames(const tfa_plan* plan, int64_t num_samples, int64_t* n_frames) {
  if (!plan || !n_frames || plan->d.kind != TFA_KIND_STFT) return fail(TFA_ERR_INVALID, "not an STFT plan");
  const int64_t n_fft = plan->d.n;
  const int64_t padded = (plan->d.flags & TFA_STFT_CENTER) ? num_samples + 2 * (n_fft / 2) : num_samples;
  if (padded < n_fft) return fail(TFA_ERR_INVALID, "signal shorter than n_fft");
  *n_frames = 1 + (padded - n_fft) / plan->d.hop;
  return TFA_OK;
}

int tfa_stft_execute(const tfa_plan* plan, int64_t batch, int64_t num_samples, const float* signal,
                     const float* window, float* out_re, float* out_im, tfa_stream stream) {
  if (!plan || plan->d.kind != TFA_KIND_STFT) return fail(TFA_ERR_INVALID, "not an STFT plan");
  if (batch < 0) return fail(TFA_ERR_INVALID, "negative batch");
  if (batch == 0) return TFA_OK;
  if (!signal || !window || !out_re || !out_im) return fail(TFA_ERR_INVALID, "null data pointer");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != plan->device)
    return fail(TFA_ERR_INVALID, "plan was created on another device than the current one");
  note_capture(plan, stream);
  const int64_t n_fft = plan->d.n;
  const bool center = plan->d.flags & TFA_STFT_CENTER;
  const int64_t pad = center ? n_fft / 2 : 0;
  if (center && num_samples <= pad) return fail(TFA_ERR_INVALID, "reflect padding needs more samples than n_fft/2");
  if (num_samples > INT32_MAX / 2) return fail(TFA_ERR_UNSUPPORTED, "signal too long");
  int64_t frames = 0;
  int rc = tfa_stft_frames(plan, num_samples, &frames);
  if (rc) return rc;
  const int n_bins = (plan->d.flags & TFA_STFT_ONESIDED) ? (int)(n_fft / 2 + 1) : (int)n_fft;
  // the kernels address a signal's output planes with 32-bit byte offsets
  if ((int64_t)n_bins * frames > (int64_t)1 << 30) return fail(TFA_ERR_UNSUPPORTED, "signal too long");
  const float scale = (plan->d.flags & TFA_STFT_NORMALIZED) ? (float)(1.0 / std::sqrt((double)n_fft)) : 1.0f;
  // a hop beyond the padded signal leaves one frame, whatever its value: keep it within int
  const int64_t hop = std::min<int64_t>(plan->d.hop, num_samples + 2 * pad);
  tfa::StftArgs a{signal, window, out_re, out_im, plan->fwd.tw, (int)num_samples, (int)hop,
                  (int)pad, (int)frames, n_bins, batch, scale, static_cast<hipStream_t>(stream)};
  a.frames_major = (plan->d.flags & TFA_STFT_FRAMES_MAJOR) != 0;
  if (!is_pow2(n_fft)) {
    a.tw_i = plan->inv.tw;
    a.chirp = plan->chirp;
    a.hs = plan->hs;
    a.m = (int)plan->m;
  }
  hipError_t e = tfa::launch_stft((int)n_fft, a);
  return e == hipSuccess ? TFA_OK : hip_fail(e, "stft launch");
}

// the inverse-STFT kernels' four-samples-per-thread output path: whole 16-byte groups everywhere
static bool vec4_ok(const tfa::IstftArgs& a, const float* out) {
  return a.hop % 4 == 0 && a.start % 4 == 0 && a.out_pitch % 4 == 0 && a.write_len % 4 == 0 &&
         (reinterpret_cast<uintptr_t>(out) & 15) == 0;
}

int tfa_istft_length(const tfa_plan* plan, int64_t n_frames, int64_t length, int64_t* out_len) {
  if (!plan || !out_len || plan->d.kind != TFA_KIND_STFT || !plan->d.inverse)
    return fail(TFA_ERR_INVALID, "not an inverse STFT plan");
  if (n_frames < 1) return fail(TFA_ERR_INVALID, "need at least one frame");
  const int64_t n_fft = plan->d.n;
  const int64_t pad = (plan->d.flags & TFA_STFT_CENTER) ? n_fft / 2 : 0;
  int64_t cur = n_fft + (n_frames - 1) * plan->d.hop - pad;
  if (pad && cur > pad && length < 0) cur -= pad;
  *out_len = length >= 0 ? length : cur;
  return TFA_OK;
}

int tfa_istft_execute(const tfa_plan* plan, int64_t batch, int64_t n_frames, const float* spec_re,
                      const float* spec_im, const float* window, float* out, int64_t length, tfa_stream stream) {
  if (!plan || plan->d.kind != TFA_KIND_STFT || !plan->d.inverse) return fail(TFA_ERR_INVALID, "not an inverse STFT plan");
  if (batch < 0) return fail(TFA_ERR_INVALID, "negative batch");
  if (batch == 0) return TFA_OK;
  if (!spec_re || !spec_im || !window || !out) return fail(TFA_ERR_INVALID, "null data pointer");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != plan->device)
    return fail(TFA_ERR_INVALID, "plan was created on another device than the current one");
  note_capture(plan, stream);
  int64_t out_len = 0;
  int rc = tfa_istft_length(plan, n_frames, length, &out_len);
  if (rc) return rc;
  const int64_t n_fft = plan->d.n, hop = plan->d.hop;
  const bool two_sided = !(plan->d.flags & TFA_STFT_ONESIDED);
  const int64_t expected = n_fft + (n_frames - 1) * hop;
  if (expected > INT32_MAX / 2 || n_frames > INT32_MAX / 2 || out_len > INT32_MAX / 2 ||
      (two_sided ? n_fft : n_fft / 2 + 1) * n_frames > INT32_MAX)
    return fail(TFA_ERR_UNSUPPORTED, "signal too long");
  const int64_t start = (plan->d.flags & TFA_STFT_CENTER) ? n_fft / 2 : 0;
  int64_t cur = expected - start;
  if (start && cur > start && length < 0) cur -= start;
  const double sc = (plan->d.flags & TFA_STFT_NORMALIZED) ? std::sqrt((double)n_fft) / (double)n_fft : 1.0 / (double)n_fft;
  tfa::IstftArgs a{spec_re, spec_im, window, out, plan->inv.tw, (int)n_frames, (int)hop, (int)((n_fft - 1) / hop),
                   batch, expected, start, cur < out_len ? cur : out_len, out_len, (float)sc,
                   static_cast<hipStream_t>(stream)};
  a.vec4 = vec4_ok(a, out);
  a.frames_major = (plan->d.flags & TFA_STFT_FRAMES_MAJOR) != 0;
  a.two_sided = two_sided;
  hipError_t e;
  if (!is_pow2(n_fft)) {
    a.blue_tw_f = plan->fwd.tw;
    a.blue_tw_i = plan->inv.tw;
    a.chirp = plan->chirp;
    a.hs = plan->hs;
    a.m = (int)plan->m;
    e = tfa::launch_istft_blue((int)n_fft, a);
  } else {
    e = tfa::launch_istft((int)n_fft, a);
  }
  return e == hipSuccess ? TFA_OK : hip_fail(e, "istft launch");
}

int tfa_stft_backward_execute(const tfa_plan* plan, int64_t batch, int64_t n_frames, const float* grad_re,
                              const float* grad_im, const float* window, float* grad_padded, int64_t padded_len,
                              tfa_stream stream) {
  if (!plan || plan->d.kind != TFA_KIND_STFT || plan->d.inverse)
    return fail(TFA_ERR_INVALID, "the STFT backward runs on the forward STFT plan");
  if (!(plan->d.flags & TFA_STFT_ONESIDED)) return fail(TFA_ERR_UNSUPPORTED, "the fused STFT backward takes onesided spectra");
  if (batch < 0) return fail(TFA_ERR_INVALID, "negative batch");
  const int64_t n_fft = plan->d.n, hop = plan->d.hop;
  const bool pow2 = is_pow2(n_fft);
  // the adjoint kernels tile like the inverse ones: a halo of floor((n-1)/hop) recomputed frames
  const int64_t halo = (n_fft - 1) / hop;
  if (pow2 ? halo >= tfa::istft_frames_per_tile((int)n_fft) : 2 * halo > tfa::stft_blue_adj_frames((int)plan->m))
    return fail(TFA_ERR_UNSUPPORTED, "hop_length too small for the fused STFT backward tile");
  if (batch == 0) return TFA_OK;
  if (!grad_re || !grad_im || !window || !grad_padded) return fail(TFA_ERR_INVALID, "null data pointer");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != plan->device)
    return fail(TFA_ERR_INVALID, "plan was created on another device than the current one");
  if (n_frames < 1) return fail(TFA_ERR_INVALID, "need at least one frame");
  // frames n_fft + (n_frames - 1) * hop long reach into the padded signal; the rest has no gradient
  const int64_t covered = n_fft + (n_frames - 1) * hop;
  if (covered > padded_len || n_frames != 1 + (padded_len - n_fft) / hop)
    return fail(TFA_ERR_INVALID, "n_frames does not match padded_len");
  if (padded_len > INT32_MAX / 2 || (n_fft / 2 + 1) * n_frames > INT32_MAX)
    return fail(TFA_ERR_UNSUPPORTED, "signal too long");
  note_capture(plan, stream);
  const double norm = (plan->d.flags & TFA_STFT_NORMALIZED) ? 1.0 / std::sqrt((double)n_fft) : 1.0;
  // power of two: r2c adjoint = interior bins halved (scale 1/2, bins 0 and n/2 doubled in the kernel)
  tfa::IstftArgs a{grad_re, grad_im, window, grad_padded, plan->inv.tw, (int)n_frames, (int)hop, (int)halo,
                   batch, covered, 0, covered, padded_len, (float)(pow2 ? 0.5 * norm : norm),
                   static_cast<hipStream_t>(stream)};
  a.adjoint = true;
  a.vec4 = vec4_ok(a, grad_padded);
  a.frames_major = (plan->d.flags & TFA_STFT_FRAMES_MAJOR) != 0;
  hipError_t e;
  if (pow2) {
    e = tfa::launch_istft((int)n_fft, a);
  } else {
    a.blue_tw_f = plan->fwd.tw;
    a.blue_tw_i = plan->inv.tw;
    a.chirp = plan->chirp;
    a.hs = plan->stft_hs_adj;
    a.m = (int)plan->m;
    e = tfa::launch_istft_blue((int)n_fft, a);
  }
  return e == hipSuccess ? TFA_OK : hip_fail(e, "stft backward launch");
}

int tfa_complex_gemm_ex(int64_t m, int64_t n, int64_t k, const float* a_re, const float* a_im, int64_t lda,
                        int32_t a_op, const float* b_re, const float* b_im, int64_t ldb, int32_t b_op, float alpha,
                        const float* bias_re, const float* bias_im, float* c_re, float* c_im, int64_t ldc,
                        tfa_stream stream) {
  if (m < 0 || n < 0 || k < 0) return fail(TFA_ERR_INVALID, "negative dimension");
  if (a_op < TFA_OP_N || a_op > TFA_OP_R || b_op < TFA_OP_N || b_op > TFA_OP_R)
    return fail(TFA_ERR_INVALID, "operand op must be TFA_OP_N, _T, _C or _R");
  if (m == 0 || n == 0) return TFA_OK;
  if (!a_re || !a_im || !b_re || !b_im || !c_re || !c_im) return fail(TFA_ERR_INVALID, "null data pointer");
  if ((bias_re == nullptr) != (bias_im == nullptr)) return fail(TFA_ERR_INVALID, "bias needs both planes or neither");
  const bool at = a_op == TFA_OP_T || a_op == TFA_OP_C, bt = b_op == TFA_OP_T || b_op == TFA_OP_C;
  // stored shapes: A is (m, k) or (k, m) when transposed; B is (k, n) or (n, k) when transposed
  if (lda < (at ? m : k) || ldb < (bt ? k : n) || ldc < n) return fail(TFA_ERR_INVALID, "leading dimension too small");
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return fail(TFA_ERR_UNSUPPORTED, "dimension above 2^31");
  tfa::GemmArgs g{m, n, k, a_re, a_im, lda, a_op, b_re, b_im, ldb, b_op, bias_re, bias_im,
                  c_re, c_im, ldc, alpha, static_cast<hipStream_t>(stream)};
  hipError_t e = tfa::launch_cgemm(g);
  return e == hipSuccess ? TFA_OK : hip_fail(e, "complex gemm launch");
}

int tfa_complex_gemm_batched(int64_t batch, int64_t m, int64_t n, int64_t k, const float* a_re, const float* a_im,
                             int64_t lda, int64_t stride_a, int32_t a_op, const float* b_re, const float* b_im,
                             int64_t ldb, int64_t stride_b, int32_t b_op, float alpha, const float* bias_re,
                             const float* bias_im, float* c_re, float* c_im, int64_t ldc, int64_t stride_c,
                             tfa_stream stream) {
  if (batch < 0 || m < 0 || n < 0 || k < 0) return fail(TFA_ERR_INVALID, "negative dimension");
  if (stride_a < 0 || stride_b < 0 || stride_c < 0) return fail(TFA_ERR_INVALID, "negative batch stride");
  if (a_op < TFA_OP_N || a_op > TFA_OP_R || b_op < TFA_OP_N || b_op > TFA_OP_R)
    return fail(TFA_ERR_INVALID, "operand op must be TFA_OP_N, _T, _C or _R");
  if (batch == 0 || m == 0 || n == 0) return TFA_OK;
  if (!a_re || !a_im || !b_re || !b_im || !c_re || !c_im) return fail(TFA_ERR_INVALID, "null data pointer");
  if ((bias_re == nullptr) != (bias_im == nullptr)) return fail(TFA_ERR_INVALID, "bias needs both planes or neither");
  const bool at = a_op == TFA_OP_T || a_op == TFA_OP_C, bt = b_op == TFA_OP_T || b_op == TFA_OP_C;
  if (lda < (at ? m : k) || ldb < (bt ? k : n) || ldc < n) return fail(TFA_ERR_INVALID, "leading dimension too small");
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return fail(TFA_ERR_UNSUPPORTED, "dimension above 2^31");
  // distinct outputs per batch entry: C's batch stride must cover one (m, ldc) matrix
  if (batch > 1 && stride_c < (m - 1) * ldc + n) return fail(TFA_ERR_INVALID, "output batch stride overlaps matrices");
  tfa::GemmArgs g{m, n, k, a_re, a_im, lda, a_op, b_re, b_im, ldb, b_op, bias_re, bias_im,
                  c_re, c_im, ldc, alpha, static_cast<hipStream_t>(stream)};
  g.batch = batch;
  g.sa = stride_a;
  g.sb = stride_b;
  g.sc = stride_c;
  hipError_t e = tfa::launch_cgemm(g);
  return e == hipSuccess ? TFA_OK : hip_fail(e, "batched complex gemm launch");
}

int tfa_complex_gemm(int64_t m, int64_t n, int64_t k, const float* a_re, const float* a_im,
                     int64_t lda, const float* b_re, const float* b_im, int64_t ldb, int32_t b_trans,
                     const float* bias_re, const float* bias_im, float* c_re, float* c_im,
                     int64_t ldc, tfa_stream stream) {
  return tfa_complex_gemm_ex(m, n, k, a_re, a_im, lda, TFA_OP_N, b_re, b_im, ldb, b_trans ? TFA_OP_T : TFA_OP_N,
                             1.0f, bias_re, bias_im, c_re, c_im, ldc, stream);
}

}  // extern "C"
