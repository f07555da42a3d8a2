// Device building blocks: complex helpers, in-register small DFTs and the LDS-resident
// Stockham transform used by every FFT kernel in this library.
//
// Conventions: DIR = -1 is the forward transform (W = exp(-2*pi*i/N)), DIR = +1 the inverse
// (unscaled; callers apply 1/N).  A transform of length N held by T = N/E threads keeps
// x[tid + T*e] in register e of thread tid on entry and X[tid + T*e] there on exit.
#pragma once
#include <hip/hip_runtime.h>

#include "fft_shape.h"

namespace tfa {

__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }

// a * (DIR * i)
template <int DIR>
__device__ __forceinline__ float2 mul_diri(float2 a) {
  return DIR < 0 ? make_float2(a.y, -a.x) : make_float2(-a.y, a.x);
}

// constexpr sin/cos (Taylor series after reduction to [-pi/4, pi/4]); used only to fold
// compile-time twiddle constants of the in-register DFTs.
constexpr double kPi = 3.14159265358979323846264338327950288;
constexpr double taylor_sin(double x) {
  double term = x, sum = x;
  for (int k = 1; k < 14; ++k) {
    term *= -x * x / ((2 * k) * (2 * k + 1));
    sum += term;
  }
  return sum;
}
constexpr double taylor_cos(double x) {
  double term = 1.0, sum = 1.0;
  for (int k = 1; k < 14; ++k) {
    term *= -x * x / ((2 * k - 1) * (2 * k));
    sum += term;
  }
  return sum;
}
// cos(2*pi*k/r), sin(2*pi*k/r) for integer k, r: reduce by octant so the series converges fast.
constexpr double cos2pi(int k, int r) {
  k = ((k % r) + r) % r;
  // angle = 2*pi*k/r in [0, 2*pi); use symmetry on 8*k/r
  double a = 2.0 * kPi * k / r;
  if (a > kPi) a -= 2.0 * kPi;
  double s = 1.0;
  if (a > kPi / 2) { a = kPi - a; s = -1.0; }
  else if (a < -kPi / 2) { a = -kPi - a; s = -1.0; }
  return s * taylor_cos(a);
}
constexpr double sin2pi(int k, int r) {
  k = ((k % r) + r) % r;
  double a = 2.0 * kPi * k / r;
  if (a > kPi) a -= 2.0 * kPi;
  if (a > kPi / 2) a = kPi - a;
  else if (a < -kPi / 2) a = -kPi - a;
  return taylor_sin(a);
}

// v * W_R^K with W_R = exp(DIR*2*pi*i/R); trivial angles use adds/negations only.
template <int K, int R, int DIR>
__device__ __forceinline__ float2 twiddle_const(float2 v) {
  constexpr int k = ((K % R) + R) % R;
  if constexpr (k == 0) {
    return v;
  } else if constexpr (2 * k == R) {
    return make_float2(-v.x, -v.y);
  } else if constexpr (4 * k == R) {
    return mul_diri<DIR>(v);
  } else if constexpr (4 * k == 3 * R) {
    return mul_diri<-DIR>(v);
  } else if constexpr (8 * k == R || 8 * k == 3 * R || 8 * k == 5 * R || 8 * k == 7 * R) {
    constexpr float h = 0.707106781186547524400844362104849f;
    constexpr float c = (8 * k == R || 8 * k == 7 * R) ? h : -h;
    constexpr float s = (float)DIR * ((8 * k == R || 8 * k == 3 * R) ? h : -h);
    // (c + i s)(x + i y) with |c| = |s| = h: h-scaled sums
    if constexpr (c > 0 && s > 0) return make_float2((v.x - v.y) * h, (v.x + v.y) * h);
    else if constexpr (c > 0 && s < 0) return make_float2((v.x + v.y) * h, (v.y - v.x) * h);
    else if constexpr (c < 0 && s > 0) return make_float2(-(v.x + v.y) * h, (v.x - v.y) * h);
    else return make_float2((v.y - v.x) * h, -(v.x + v.y) * h);
  } else {
    constexpr float c = (float)cos2pi(k, R);
    constexpr float s = (float)((double)DIR * sin2pi(k, R));
    return make_float2(v.x * c - v.y * s, v.x * s + v.y * c);
  }
}

// In-register DFT of length R on a[0..R) (natural order in and out).
template <int R, int DIR>
struct Dft;

template <int DIR>
struct Dft<1, DIR> {
  __device__ __forceinline__ static void run(float2*) {}
};

template <int DIR>
struct Dft<2, DIR> {
  __device__ __forceinline__ static void run(float2* a) {
    float2 t = a[0];
    a[0] = cadd(t, a[1]);
    a[1] = csub(t, a[1]);
  }
};

template <int DIR>
struct Dft<4, DIR> {
  __device__ __forceinline__ static void run(float2* a) {
    float2 t0 = cadd(a[0], a[2]);
    float2 t1 = csub(a[0], a[2]);
    float2 t2 = cadd(a[1], a[3]);
    float2 t3 = mul_diri<DIR>(csub(a[1], a[3]));
    a[0] = cadd(t0, t2);
    a[2] = csub(t0, t2);
    a[1] = cadd(t1, t3);
    a[3] = csub(t1, t3);
  }
};

// Radix 3: a0 + a1 + a2, and a0 - (a1 + a2)/2 -/+ (sqrt(3)/2) (DIR i)(a1 - a2) for outputs 1, 2.
template <int DIR>
struct Dft<3, DIR> {
  __device__ __forceinline__ static void run(float2* a) {
    constexpr float s3 = 0.866025403784438646763723170752936f;
    const float2 t1 = cadd(a[1], a[2]);
    const float2 t2 = make_float2(a[0].x - 0.5f * t1.x, a[0].y - 0.5f * t1.y);
    const float2 t3 = cscale(mul_diri<DIR>(csub(a[1], a[2])), s3);
    a[0] = cadd(a[0], t1);
    a[1] = cadd(t2, t3);
    a[2] = csub(t2, t3);
  }
};

// R = R1 * R2: DFT_R2 over the stride-R1 subsequences, twiddle W_R^{l q}, then DFT_R1.
template <int R1, int R2, int DIR>
struct DftSplit {
  static constexpr int R = R1 * R2;
  template <int L, int Q>
  __device__ __forceinline__ static void tw(float2 (&b)[R1][R2]) {
    if constexpr (L < R1) {
      if constexpr (Q < R2) {
        b[L][Q] = twiddle_const<L * Q, R, DIR>(b[L][Q]);
        tw<L, Q + 1>(b);
      } else {
        tw<L + 1, 0>(b);
      }
    }
  }
  __device__ __forceinline__ static void run(float2* a) {
    float2 b[R1][R2];
#pragma unroll
    for (int l = 0; l < R1; ++l) {
#pragma unroll
      for (int m = 0; m < R2; ++m) b[l][m] = a[l + R1 * m];
      Dft<R2, DIR>::run(b[l]);
    }
    tw<0, 0>(b);
#pragma unroll
    for (int q = 0; q < R2; ++q) {
      float2 c[R1];
#pragma unroll
      for (int l = 0; l < R1; ++l) c[l] = b[l][q];
      Dft<R1, DIR>::run(c);
#pragma unroll
      for (int p = 0; p < R1; ++p) a[q + R2 * p] = c[p];
    }
  }
};

template <int DIR>
struct Dft<8, DIR> {
  __device__ __forceinline__ static void run(float2* a) { DftSplit<2, 4, DIR>::run(a); }
};
template <int DIR>
struct Dft<16, DIR> {
  __device__ __forceinline__ static void run(float2* a) { DftSplit<4, 4, DIR>::run(a); }
};
template <int DIR>
struct Dft<32, DIR> {
  __device__ __forceinline__ static void run(float2* a) { DftSplit<4, 8, DIR>::run(a); }
};
// radices with a factor 3 (mixed-radix lengths 3 * 2^k and 9 * 2^k)
template <int DIR>
struct Dft<6, DIR> {
  __device__ __forceinline__ static void run(float2* a) { DftSplit<2, 3, DIR>::run(a); }
};
template <int DIR>
struct Dft<12, DIR> {
  __device__ __forceinline__ static void run(float2* a) { DftSplit<4, 3, DIR>::run(a); }
};
template <int DIR>
struct Dft<24, DIR> {
  __device__ __forceinline__ static void run(float2* a) { DftSplit<8, 3, DIR>::run(a); }
};

// Synchronisation between the LDS write and read halves of a pass exchange.  When a transform
// lives inside one wavefront (T <= 64) program order within the wave suffices and only the
// compiler must be kept from moving LDS accesses across the exchange.
template <bool WAVE_LOCAL>
__device__ __forceinline__ void exchange_sync() {
  if constexpr (WAVE_LOCAL) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    __syncthreads();
  }
}

// LDS-resident Stockham FFT of one length-N transform held by T = N/E threads.
//   v:    registers, x[tid + T*e] on entry, X[tid + T*e] on exit
//   lre/lim: this transform's LDS scratch, lds_pad(N) floats each
//   tw:   the plan's twiddle table for (N, E, DIR) (layout from make_shape)
// SPLIT: exchange the real and imaginary planes one after the other through `lre` alone (lim
// unused): half the LDS per transform, twice the synchronisations.
// IL: `lre` holds lds_pad(N) interleaved float2 (re, im) entries (lim unused): one 64-bit LDS
// access per element instead of two 32-bit ones (gfx950 serves a 64-lane ds_read_b64 of
// consecutive float2 in the cycles of a ds_read_b32, so this halves LDS time as well).
// PF: each pass requests the next pass's twiddles before its exchange barriers, so their table
// latency overlaps the exchange instead of following it (E/2 float4 more registers live there).
// DB: double-buffered exchange (IL only): pass p writes and reads LDS buffer p % 2, the second one
// 2 * lds_pad(N) floats after `lre`, so one workgroup barrier per exchange suffices (a buffer is
// rewritten two passes later, after every thread has passed the intervening barrier, which
// follows its reads of that buffer); run() starts with a barrier so that back-to-back transforms
// in one kernel do not overwrite a buffer another thread is still reading.  Nothing after run()
// may use the LDS without its own barrier.
template <int N, int E, int DIR, bool WAVE_LOCAL, bool SPLIT = false, bool IL = false, bool PF = false,
          bool DB = false>
struct LdsFft {
  static constexpr LdsShape S = make_shape(N, E);
  static constexpr int T = N / E;
  static_assert(!DB || (IL && !SPLIT && !WAVE_LOCAL), "double buffering is for the interleaved workgroup exchange");
  // consecutive T-thread transforms stay inside one wavefront only when T divides 64
  static_assert(!WAVE_LOCAL || 64 % T == 0, "a wave-local transform must not straddle wavefronts");
  static constexpr int DBOFF = 2 * lds_pad(N);  // floats between the two buffers
  static constexpr int TQ = PF ? (E / 2 > 0 ? E / 2 : 1) : 1;  // float4 twiddles per thread per pass

  template <int P>
  __device__ __forceinline__ static void pass(float2 (&v)[E], float* lre, float* lim,
                                              const float2* __restrict__ tw, int tid, const float4 (&tc)[TQ]) {
    if constexpr (P < S.npass) {
      constexpr int R = S.radix[P];
      constexpr int NB = E / R;
      static_assert(E % R == 0, "each pass radix must divide the elements per thread");
      static_assert(P == 0 || R % 2 == 0, "twiddled passes read their table as float4 pairs (even radix)");
      constexpr int LS = S.ls[P];
      constexpr bool LAST = (P == S.npass - 1);
      // the pass's LDS write index is linear in u when the radix (first pass) or the span LS
      // (later passes) is a multiple of the 16-word padding period
      constexpr bool LIN_W = (LS == 1) ? (R % 16 == 0) : (LS % 16 == 0);
      float2 w[NB][R];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int j = tid + b * T;
        const int k = (int)((unsigned)j % (unsigned)LS);
#pragma unroll
        for (int r = 0; r < R; ++r) w[b][r] = v[b + r * NB];
        if constexpr (P > 0) {
          const float4* t4 = reinterpret_cast<const float4*>(tw + S.twoff[P] + k * R);
#pragma unroll
          for (int r2 = 0; r2 < R / 2; ++r2) {
            float4 q = PF ? tc[PF ? b * (R / 2) + r2 : 0] : t4[r2];
            if (r2 > 0) w[b][2 * r2] = cmul(w[b][2 * r2], make_float2(q.x, q.y));
            w[b][2 * r2 + 1] = cmul(w[b][2 * r2 + 1], make_float2(q.z, q.w));
          }
        }
        Dft<R, DIR>::run(w[b]);
        if constexpr (LAST) {
#pragma unroll
          for (int u = 0; u < R; ++u) v[b + u * NB] = w[b][u];
        } else if constexpr (!SPLIT) {
          store_pass<R, LS, LIN_W>(w[b], (DB && (P & 1)) ? lre + DBOFF : lre, lim, j, k, IL ? 3 : 2);
        }
      }
      if constexpr (!LAST) {
        float4 tn[TQ];
        if constexpr (PF) {
          constexpr int R1 = S.radix[P + 1], NB1 = E / R1, LS1 = S.ls[P + 1];
#pragma unroll
          for (int b = 0; b < NB1; ++b) {
            const int k1 = (int)((unsigned)(tid + b * T) % (unsigned)LS1);
            const float4* t4 = reinterpret_cast<const float4*>(tw + S.twoff[P + 1] + k1 * R1);
#pragma unroll
            for (int r2 = 0; r2 < R1 / 2; ++r2) tn[b * (R1 / 2) + r2] = t4[r2];
          }
        }
        if constexpr (!SPLIT) {
          exchange_sync<WAVE_LOCAL>();
          load_pass(v, (DB && (P & 1)) ? lre + DBOFF : lre, lim, tid, IL ? 3 : 2);
          if constexpr (!DB) exchange_sync<WAVE_LOCAL>();
        } else {
#pragma unroll
          for (int plane = 0; plane < 2; ++plane) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              const int j = tid + b * T;
              store_pass<R, LS, LIN_W>(w[b], lre, lre, j, (int)((unsigned)j % (unsigned)LS), plane);
            }
            exchange_sync<WAVE_LOCAL>();
            load_pass(v, lre, lre, tid, plane);
            exchange_sync<WAVE_LOCAL>();
          }
        }
        pass<P + 1>(v, lre, lim, tw, tid, tn);
      }
    }
  }

  // which: 0 = real plane into a, 1 = imaginary plane into a, 2 = real into a and imag into b,
  //        3 = interleaved float2 entries in a
  template <int R, int LS, bool LIN_W>
  __device__ __forceinline__ static void store_pass(const float2 (&w)[R], float* a, float* b, int j, int k,
                                                    int which) {
    if constexpr (LIN_W) {
      // padded index = base + compile-time offset per u (immediate-offset LDS stores)
      const int base = LS == 1 ? j * (R + R / 16) : lds_pad((j - k) * R) + k + (k >> 4);
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const int off = LS == 1 ? u + (u >> 4) : u * (LS + LS / 16);
        if (which == 3) {
          reinterpret_cast<float2*>(a)[base + off] = w[u];
        } else if (which == 2) {
          a[base + off] = w[u].x;
          b[base + off] = w[u].y;
        } else {
          a[base + off] = which ? w[u].y : w[u].x;
        }
      }
    } else {
      const int base = (j - k) * R + k;
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const int idx = lds_pad(base + u * LS);
        if (which == 3) {
          reinterpret_cast<float2*>(a)[idx] = w[u];
        } else if (which == 2) {
          a[idx] = w[u].x;
          b[idx] = w[u].y;
        } else {
          a[idx] = which ? w[u].y : w[u].x;
        }
      }
    }
  }

  __device__ __forceinline__ static void load_pass(float2 (&v)[E], const float* a, const float* b, int tid,
                                                   int which) {
    if constexpr (T % 16 == 0) {
      const int rb = tid + (tid >> 4);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int idx = rb + e * (T + T / 16);
        if (which == 3) v[e] = reinterpret_cast<const float2*>(a)[idx];
        else if (which == 2) v[e] = make_float2(a[idx], b[idx]);
        else if (which == 0) v[e].x = a[idx];
        else v[e].y = a[idx];
      }
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int idx = lds_pad(tid + T * e);
        if (which == 3) v[e] = reinterpret_cast<const float2*>(a)[idx];
        else if (which == 2) v[e] = make_float2(a[idx], b[idx]);
        else if (which == 0) v[e].x = a[idx];
        else v[e].y = a[idx];
      }
    }
  }

  __device__ __forceinline__ static void run(float2 (&v)[E], float* lre, float* lim,
                                             const float2* __restrict__ tw, int tid) {
    const float4 none[TQ] = {};
    if constexpr (DB) exchange_sync<false>();
    pass<0>(v, lre, lim, tw, tid, none);
  }
};

// M independent wave-local transforms of length N per thread group (interleaved LDS exchange),
// advanced pass by pass together: one exchange synchronisation per pass for all of them, so a
// wavefront has M times the independent work between exchanges.  area[m] is transform m's LDS
// scratch (lds_pad(N) float2 entries); v[m] as LdsFft's v.
template <int N, int E, int DIR, int M>
struct LdsFftMulti {
  using F = LdsFft<N, E, DIR, true, false, true, false>;
  static constexpr LdsShape S = F::S;
  static constexpr int T = F::T;

  template <int P>
  __device__ __forceinline__ static void pass(float2 (&v)[M][E], float* const (&area)[M],
                                              const float2* __restrict__ tw, int tid) {
    if constexpr (P < S.npass) {
      constexpr int R = S.radix[P];
      constexpr int NB = E / R;
      constexpr int LS = S.ls[P];
      constexpr bool LAST = (P == S.npass - 1);
      constexpr bool LIN_W = (LS == 1) ? (R % 16 == 0) : (LS % 16 == 0);
#pragma unroll
      for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int j = tid + b * T;
          const int k = (int)((unsigned)j % (unsigned)LS);
          float2 w[R];
#pragma unroll
          for (int r = 0; r < R; ++r) w[r] = v[m][b + r * NB];
          if constexpr (P > 0) {
            const float4* t4 = reinterpret_cast<const float4*>(tw + S.twoff[P] + k * R);
#pragma unroll
            for (int r2 = 0; r2 < R / 2; ++r2) {
              const float4 q = t4[r2];
              if (r2 > 0) w[2 * r2] = cmul(w[2 * r2], make_float2(q.x, q.y));
              w[2 * r2 + 1] = cmul(w[2 * r2 + 1], make_float2(q.z, q.w));
            }
          }
          Dft<R, DIR>::run(w);
          if constexpr (LAST) {
#pragma unroll
            for (int u = 0; u < R; ++u) v[m][b + u * NB] = w[u];
          } else {
            F::template store_pass<R, LS, LIN_W>(w, area[m], nullptr, j, k, 3);
          }
        }
      }
      if constexpr (!LAST) {
        exchange_sync<true>();
#pragma unroll
        for (int m = 0; m < M; ++m) F::load_pass(v[m], area[m], nullptr, tid, 3);
        exchange_sync<true>();
        pass<P + 1>(v, area, tw, tid);
      }
    }
  }

  __device__ __forceinline__ static void run(float2 (&v)[M][E], float* const (&area)[M],
                                             const float2* __restrict__ tw, int tid) {
    pass<0>(v, area, tw, tid);
  }
};

}  // namespace tfa
