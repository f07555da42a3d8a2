// Complex GEMM on the fp32 matrix cores (v_mfma_f32_32x32x2f32), split re/im planes.
//
//   C = alpha * (op(A) @ op(B)) + bias,  op(X) = X, X^T, conj(X)^T or conj(X)
//   C_re = A_re B_re - A_im B_im,  C_im = A_re B_im + A_im B_re   (on the op'ed operands)
// A transposed operand is staged through LDS in the same [k][i] layout as a plain one (only the
// global load pattern differs); conjugation negates the imaginary plane as it is staged.
//
// One kernel computes all four real products: each k-step loads the A_re/A_im and B_re/B_im
// fragments once from LDS and issues four MFMAs into two accumulator sets (the NKI kernel's
// "stationary reuse" idea, trnfft/nki/dispatch.py:121-200 and :267-345, in CDNA4 form).
// Workgroup tile 128 x 128 (per plane), 4 waves of 64 x 64, BK = 16 k per LDS stage with the
// next stage prefetched into registers while the current one is consumed.
#include <algorithm>

#include "kernels.h"

namespace tfa {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 128, GBK = 16;
constexpr int GLD = GBM + 2;  // LDS row pitch in floats (pad 2: transposed stores hit distinct banks)

// Global -> register tile loads. A tile: GBM rows x GBK k (k contiguous in memory). Thread t
// covers row t/2, k offset (t%2)*8: 8 floats per plane.
struct ATile {
  float re[8], im[8];
};

__device__ __forceinline__ void load_kmajor_tile(const float* __restrict__ P_re, const float* __restrict__ P_im,
                                                 long long ld, int rows, int K, int row0, int k0, int t,
                                                 bool vec_ok, ATile& o) {
  const int r = row0 + t / 2;
  const int kq = k0 + (t % 2) * 8;
  if (r < rows && vec_ok && kq + 8 <= K) {
    const float4* pr = reinterpret_cast<const float4*>(P_re + (size_t)r * ld + kq);
    const float4* pi = reinterpret_cast<const float4*>(P_im + (size_t)r * ld + kq);
    float4 a = pr[0], b = pr[1], c = pi[0], d = pi[1];
    o.re[0] = a.x; o.re[1] = a.y; o.re[2] = a.z; o.re[3] = a.w;
    o.re[4] = b.x; o.re[5] = b.y; o.re[6] = b.z; o.re[7] = b.w;
    o.im[0] = c.x; o.im[1] = c.y; o.im[2] = c.z; o.im[3] = c.w;
    o.im[4] = d.x; o.im[5] = d.y; o.im[6] = d.z; o.im[7] = d.w;
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const bool in = r < rows && kq + c < K;
      o.re[c] = in ? P_re[(size_t)r * ld + kq + c] : 0.0f;
      o.im[c] = in ? P_im[(size_t)r * ld + kq + c] : 0.0f;
    }
  }
}

// B tile for the non-transposed case: GBK k-rows x GBN columns (n contiguous). Thread t covers
// k row t/16, columns (t%16)*8 .. +8.
__device__ __forceinline__ void load_nmajor_tile(const float* __restrict__ P_re, const float* __restrict__ P_im,
                                                 long long ld, int N, int K, int col0, int k0, int t,
                                                 bool vec_ok, ATile& o) {
  const int k = k0 + t / 16;
  const int j = col0 + (t % 16) * 8;
  if (k < K && vec_ok && j + 8 <= N) {
    const float4* pr = reinterpret_cast<const float4*>(P_re + (size_t)k * ld + j);
    const float4* pi = reinterpret_cast<const float4*>(P_im + (size_t)k * ld + j);
    float4 a = pr[0], b = pr[1], c = pi[0], d = pi[1];
    o.re[0] = a.x; o.re[1] = a.y; o.re[2] = a.z; o.re[3] = a.w;
    o.re[4] = b.x; o.re[5] = b.y; o.re[6] = b.z; o.re[7] = b.w;
    o.im[0] = c.x; o.im[1] = c.y; o.im[2] = c.z; o.im[3] = c.w;
    o.im[4] = d.x; o.im[5] = d.y; o.im[6] = d.z; o.im[7] = d.w;
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const bool in = k < K && j + c < N;
      o.re[c] = in ? P_re[(size_t)k * ld + j + c] : 0.0f;
      o.im[c] = in ? P_im[(size_t)k * ld + j + c] : 0.0f;
    }
  }
}

// LDS layout: S[plane][k][i] (i contiguous) so an MFMA operand fragment is 32 consecutive floats.
// `sim` (+1 or -1) multiplies the imaginary plane (conjugation).
__device__ __forceinline__ void store_kmajor(float (*S)[GBK][GLD], int t, const ATile& o, float sim) {
  const int r = t / 2, kq = (t % 2) * 8;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    S[0][kq + c][r] = o.re[c];
    S[1][kq + c][r] = o.im[c] * sim;
  }
}

__device__ __forceinline__ void store_nmajor(float (*S)[GBK][GLD], int t, const ATile& o, float sim) {
  const int k = t / 16, j = (t % 16) * 8;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    S[0][k][j + c] = o.re[c];
    S[1][k][j + c] = o.im[c] * sim;
  }
}

// Operand staging: A_T = op(A) is a transpose (A stored k x m); B_T = op(B) is a transpose
// (B stored n x k).  A plain A and a transposed B are k-contiguous; the other two m/n-contiguous.
template <bool A_T>
__device__ __forceinline__ void load_a(const float* A_re, const float* A_im, long long lda, int M, int K, int row0,
                                       int k0, int t, bool vec, ATile& o) {
  if constexpr (A_T) load_nmajor_tile(A_re, A_im, lda, M, K, row0, k0, t, vec, o);
  else load_kmajor_tile(A_re, A_im, lda, M, K, row0, k0, t, vec, o);
}
template <bool B_T>
__device__ __forceinline__ void load_b(const float* B_re, const float* B_im, long long ldb, int N, int K, int col0,
                                       int k0, int t, bool vec, ATile& o) {
  if constexpr (B_T) load_kmajor_tile(B_re, B_im, ldb, N, K, col0, k0, t, vec, o);
  else load_nmajor_tile(B_re, B_im, ldb, N, K, col0, k0, t, vec, o);
}
template <bool KMAJOR>
__device__ __forceinline__ void stage(float (*S)[GBK][GLD], int t, const ATile& o, float sim) {
  if constexpr (KMAJOR) store_kmajor(S, t, o, sim);
  else store_nmajor(S, t, o, sim);
}

template <bool A_T, bool B_T>
__global__ __launch_bounds__(256, 2) void cgemm_kernel(int M, int N, int K, const float* __restrict__ A_re,
                                                    const float* __restrict__ A_im, long long lda, float a_sim,
                                                    const float* __restrict__ B_re, const float* __restrict__ B_im,
                                                    long long ldb, float b_sim, const float* __restrict__ bias_re,
                                                    const float* __restrict__ bias_im, float* __restrict__ C_re,
                                                    float* __restrict__ C_im, long long ldc, float alpha,
                                                    long long sa, long long sb, long long sc) {
  __shared__ float As[2][GBK][GLD];
  __shared__ float Bs[2][GBK][GLD];
  // batched products: blockIdx.y selects the matrix triple (batch strides in floats; a stride of 0
  // broadcasts one operand over the batch)
  {
    const size_t bz = blockIdx.y;
    A_re += bz * sa;
    A_im += bz * sa;
    B_re += bz * sb;
    B_im += bz * sb;
    C_re += bz * sc;
    C_im += bz * sc;
  }
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = t >> 6;
  const int wm = w >> 1, wn = w & 1;
  // XCD-aware: neighbouring row tiles (which share B) run on one XCD
  const long long tiles_n = (N + GBN - 1) / GBN;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const int row0 = (int)(tile / tiles_n) * GBM;
  const int col0 = (int)(tile % tiles_n) * GBN;
  const bool a_vec = (lda % 4 == 0) && ((reinterpret_cast<size_t>(A_re) | reinterpret_cast<size_t>(A_im)) % 16 == 0);
  const bool b_vec = (ldb % 4 == 0) && ((reinterpret_cast<size_t>(B_re) | reinterpret_cast<size_t>(B_im)) % 16 == 0);

  floatx16 acc_re[2][2], acc_im[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc_re[i][j][r] = 0.0f;
        acc_im[i][j][r] = 0.0f;
      }

  ATile pa, pb;
  load_a<A_T>(A_re, A_im, lda, M, K, row0, 0, t, a_vec, pa);
  load_b<B_T>(B_re, B_im, ldb, N, K, col0, 0, t, b_vec, pb);

  const int li = lane & 31;
  const int lk = lane >> 5;
  for (int k0 = 0; k0 < K; k0 += GBK) {
    stage<!A_T>(As, t, pa, a_sim);
    stage<B_T>(Bs, t, pb, b_sim);
    __syncthreads();
    if (k0 + GBK < K) {
      load_a<A_T>(A_re, A_im, lda, M, K, row0, k0 + GBK, t, a_vec, pa);
      load_b<B_T>(B_re, B_im, ldb, N, K, col0, k0 + GBK, t, b_vec, pb);
    }
#pragma unroll
    for (int kk = 0; kk < GBK; kk += 2) {
      float ar[2], ai[2], nai[2], br[2], bi[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ar[i] = As[0][kk + lk][wm * 64 + i * 32 + li];
        ai[i] = As[1][kk + lk][wm * 64 + i * 32 + li];
        nai[i] = -ai[i];
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        br[j] = Bs[0][kk + lk][wn * 64 + j * 32 + li];
        bi[j] = Bs[1][kk + lk][wn * 64 + j * 32 + li];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc_re[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ar[i], br[j], acc_re[i][j], 0, 0, 0);
          acc_re[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(nai[i], bi[j], acc_re[i][j], 0, 0, 0);
          acc_im[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ar[i], bi[j], acc_im[i][j], 0, 0, 0);
          acc_im[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ai[i], br[j], acc_im[i][j], 0, 0, 0);
        }
    }
    __syncthreads();
  }

  // D layout of v_mfma_f32_32x32x2f32: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, col l%32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = col0 + wn * 64 + j * 32 + li;
      if (col >= N) continue;
      const float b_re = bias_re ? bias_re[col] : 0.0f;
      const float b_im = bias_im ? bias_im[col] : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = row0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (row < M) {
          C_re[(size_t)row * ldc + col] = acc_re[i][j][r] * alpha + b_re;
          C_im[(size_t)row * ldc + col] = acc_im[i][j][r] * alpha + b_im;
        }
      }
    }
}

template <bool A_T, bool B_T>
static void launch_cgemm_t(const GemmArgs& a, long long tiles) {
  const float a_sim = (a.a_op == 2 || a.a_op == 3) ? -1.0f : 1.0f;
  const float b_sim = (a.b_op == 2 || a.b_op == 3) ? -1.0f : 1.0f;
  constexpr long long kMaxGridY = 65535;
  for (long long b0 = 0; b0 < a.batch; b0 += kMaxGridY) {
    const unsigned nb = (unsigned)std::min(kMaxGridY, a.batch - b0);
    hipLaunchKernelGGL((cgemm_kernel<A_T, B_T>), dim3((unsigned)tiles, nb), dim3(256), 0, a.stream, (int)a.m,
                       (int)a.n, (int)a.k, a.a_re + b0 * a.sa, a.a_im + b0 * a.sa, a.lda, a_sim, a.b_re + b0 * a.sb,
                       a.b_im + b0 * a.sb, a.ldb, b_sim, a.bias_re, a.bias_im, a.c_re + b0 * a.sc,
                       a.c_im + b0 * a.sc, a.ldc, a.alpha, a.sa, a.sb, a.sc);
  }
}

hipError_t launch_cgemm(const GemmArgs& a) {
  const long long tiles = ((a.m + GBM - 1) / GBM) * ((a.n + GBN - 1) / GBN);
  const bool at = a.a_op == 1 || a.a_op == 2, bt = a.b_op == 1 || a.b_op == 2;
  if (at) {
    if (bt) launch_cgemm_t<true, true>(a, tiles);
    else launch_cgemm_t<true, false>(a, tiles);
  } else {
    if (bt) launch_cgemm_t<false, true>(a, tiles);
    else launch_cgemm_t<false, false>(a, tiles);
  }
  return hipGetLastError();
}

}  // namespace tfa
