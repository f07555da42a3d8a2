// Strided multi-pass FFT: a power-of-two axis of length N = L1*...*LP > 4096 (P = 2 or 3 factors)
// transformed where it lies, data viewed as (outer, N, S) row-major, S columns.  The recursive
// four-step with the factors as passes, each a strided pass through a workspace, no transposes:
//   pass p < P: for every block (o, k1..k_{p-1}) of M_{p-1} = Lp*M_p positions (M_p = L_{p+1}..LP),
//     columns col = m*S + s (m < M_p): DFT over the Lp positions n_p*M_p + m (element stride
//     M_p*S), times W_{M_{p-1}}^(m*k_p), written back in the same layout (output k_p where n_p
//     was), so the block splits into Lp blocks (o, k1..k_p) of M_p positions;
//   pass P: for every (o, k1..k_{P-1}, s), the DFT over the LP positions of block (o, k1..k_{P-1})
//     (element stride S), written to X[o][k1 + L1*k2 + ... + L1..L_{P-1}*kP][s].
// Replaces, for such axes, the transpose-copy + contiguous FFT + transpose-back of
// trnfft/api.py:496-516 (_fft_along_dim).
#include "kernels.h"

namespace tfa {

namespace {

// Addressing of one pass.  Column col = q*S + r (q = col / S); with qa = q & (2^qa_bits - 1) and
// qb = q >> qa_bits, element j of the column is read from o*blk + qa*in_a + qb*in_b + r + j*in_step
// and output k written to o*blk + qa*out_a + qb*out_b + r + k*out_step.  Twiddled passes
// multiply output k by W_N^((q*tw_mult*k) mod N) (tables W^lo, W^hi of the whole length N).
struct SfsPass {
  long long S, blk, tiles_per_block;
  long long in_a, in_b, in_step, out_a, out_b, out_step;
  int qa_bits;
  unsigned tw_mult;
  int lo_bits;
  unsigned nmask;
  float scale;
};

// bits of the column-index split that leave qb = 0 for any column index in range
constexpr int kNoSplit = 40;

}  // namespace

// A workgroup takes C adjacent columns of one block (the single-pass strided kernel's shape);
// every pass has at least 64 >= C columns per block, so every tile is whole.  The data pointers
// are not restrict: a middle pass runs in place (in == out).
template <int L, int DIR, bool REAL_IN, bool TWIDDLE, int C = fourstep_tile(L)>
__global__ __launch_bounds__(C * (L / lds_epth(L))) void strided_fs_kernel(
    const float* in_re, const float* in_im, float* out_re, float* out_im, const float2* __restrict__ tw,
    const float2* __restrict__ tw_lo, const float2* __restrict__ tw_hi, SfsPass p) {
  constexpr int E = lds_epth(L), T = L / E;
  constexpr int PADN = lds_pad(L) + 1;
  // interleaved (re, im) exchange except at 4096 (as the single-pass strided kernel)
  constexpr bool IL = L != 4096;
  __shared__ float2 lds[C * PADN];
  const int c = threadIdx.x % C;  // column within the tile (fast across lanes)
  const int t = threadIdx.x / C;
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long o = tile / p.tiles_per_block;
  const long long col = (tile % p.tiles_per_block) * C + c;
  const long long q = col / p.S, r = col - q * p.S;
  const long long qa = q & ((1LL << p.qa_bits) - 1), qb = q >> p.qa_bits;
  const size_t ib = (size_t)(o * p.blk + qa * p.in_a + qb * p.in_b + r) + (size_t)t * (size_t)p.in_step;
  const size_t istep = (size_t)T * (size_t)p.in_step;
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
    // output k = t + T*(TF*a + j): W^(g*(t + T*TF*a)) * W^(g*T*j) with g = q*tw_mult, TF-1 + E/TF
    // table pairs per thread; products mod 2^32 keep the exponent exact mod N (N | 2^32)
    constexpr int TF = E < 4 ? E : 4;
    const unsigned g = (unsigned)q * p.tw_mult;
    const unsigned lomask = (1u << p.lo_bits) - 1;
    float2 w[TF];
#pragma unroll
    for (int j = 1; j < TF; ++j) {
      const unsigned m = (g * (unsigned)(T * j)) & p.nmask;
      w[j] = cmul(tw_lo[m & lomask], tw_hi[m >> p.lo_bits]);
    }
#pragma unroll
    for (int a = 0; a < E / TF; ++a) {
      const unsigned m = (g * (unsigned)(t + T * TF * a)) & p.nmask;
      const float2 f = cmul(tw_lo[m & lomask], tw_hi[m >> p.lo_bits]);
      v[TF * a] = cmul(v[TF * a], f);
#pragma unroll
      for (int j = 1; j < TF; ++j) v[TF * a + j] = cmul(v[TF * a + j], cmul(f, w[j]));
    }
  }
  const size_t ob = (size_t)(o * p.blk + qa * p.out_a + qb * p.out_b + r) + (size_t)t * (size_t)p.out_step;
  const size_t ostep = (size_t)T * (size_t)p.out_step;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const size_t i = ob + e * ostep;
    const float2 y = TWIDDLE ? v[e] : cscale(v[e], p.scale);
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

// Last pass of a contiguous axis (S = 1): column q's LP inputs are one contiguous block, so the
// per-column loads of strided_fs_kernel would put every lane on its own block.  The workgroup's C
// blocks are loaded with lanes along the block (coalesced runs of LP floats) into the columns'
// LDS areas, then transformed and stored as there (lanes across columns: C consecutive outputs).
template <int L, int DIR, int C = fourstep_tile(L)>
__global__ __launch_bounds__(C * (L / lds_epth(L))) void strided_fs_last_contig_kernel(
    const float* in_re, const float* in_im, float* out_re, float* out_im, const float2* __restrict__ tw,
    SfsPass p) {
  constexpr int E = lds_epth(L), T = L / E, THREADS = C * T;
  constexpr int PADN = lds_pad(L) + 1;
  static_assert(L != 4096, "staged last pass uses the interleaved exchange");
  __shared__ float2 lds[C * PADN];
  const long long tile = xcd_tile_remap(blockIdx.x, gridDim.x);
  const long long o = tile / p.tiles_per_block;
  const long long q0 = (tile % p.tiles_per_block) * C;
  const long long qmask = (1LL << p.qa_bits) - 1;
  const size_t ob = (size_t)(o * p.blk);
#pragma unroll 4
  for (int i = threadIdx.x; i < C * L; i += THREADS) {
    const int c = i / L, j = i % L;
    const long long q = q0 + c;
    const size_t src = ob + (size_t)((q & qmask) * p.in_a + (q >> p.qa_bits) * p.in_b) + j;
    lds[c * PADN + lds_pad(j)] = make_float2(ld_stream(in_re + src), ld_stream(in_im + src));
  }
  __syncthreads();
  const int c = threadIdx.x % C, t = threadIdx.x / C;
  float2* base = lds + c * PADN;
  float2 v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = base[lds_pad(t + T * e)];
  __syncthreads();  // the column areas become the transforms' exchange areas
  LdsFft<L, E, DIR, false, false, true>::run(v, reinterpret_cast<float*>(base), nullptr, tw, t);
  const long long q = q0 + c;
  const size_t o0 = ob + (size_t)((q & qmask) * p.out_a + (q >> p.qa_bits) * p.out_b) + (size_t)t * (size_t)p.out_step;
  const size_t ostep = (size_t)T * (size_t)p.out_step;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float2 y = cscale(v[e], p.scale);
    st_stream(out_re + o0 + e * ostep, y.x);
    st_stream(out_im + o0 + e * ostep, y.y);
  }
}

template <int L, int DIR>
static hipError_t launch_sfs_pass_t(const float* in_re, const float* in_im, float* out_re, float* out_im,
                                    const float2* tw, const StridedFourStepArgs& a, long long blocks, bool twiddle,
                                    const SfsPass& p, hipStream_t s) {
  constexpr int C = fourstep_tile(L), TH = C * (L / lds_epth(L));
  const long long grid = blocks * p.tiles_per_block;
  if (grid > 0xffffffffLL) return hipErrorInvalidValue;
  if constexpr (L != 4096) {
    if (!twiddle && p.S == 1) {
      hipLaunchKernelGGL((strided_fs_last_contig_kernel<L, DIR>), dim3((unsigned)grid), dim3(TH), 0, s, in_re, in_im,
                         out_re, out_im, tw, p);
      return hipGetLastError();
    }
  }
  if (twiddle && in_im == nullptr)
    hipLaunchKernelGGL((strided_fs_kernel<L, DIR, true, true>), dim3((unsigned)grid), dim3(TH), 0, s, in_re, in_im,
                       out_re, out_im, tw, a.tw_lo, a.tw_hi, p);
  else if (twiddle)
    hipLaunchKernelGGL((strided_fs_kernel<L, DIR, false, true>), dim3((unsigned)grid), dim3(TH), 0, s, in_re, in_im,
                       out_re, out_im, tw, a.tw_lo, a.tw_hi, p);
  else
    hipLaunchKernelGGL((strided_fs_kernel<L, DIR, false, false>), dim3((unsigned)grid), dim3(TH), 0, s, in_re, in_im,
                       out_re, out_im, tw, a.tw_lo, a.tw_hi, p);
  return hipGetLastError();
}

// Column tile of the pass over length l (the host mirror of the template default).
static int sfs_tile(int l) { return fourstep_tile(l); }

template <int DIR>
static hipError_t launch_sfs_pass(int l, const float* in_re, const float* in_im, float* out_re, float* out_im,
                                  const float2* tw, const StridedFourStepArgs& a, long long blocks, bool twiddle,
                                  const SfsPass& p) {
  switch (l) {
#define TFA_SFS_CASE(LEN) \
  case LEN: return launch_sfs_pass_t<LEN, DIR>(in_re, in_im, out_re, out_im, tw, a, blocks, twiddle, p, a.stream);
    TFA_SFS_CASE(64)
    TFA_SFS_CASE(128)
    TFA_SFS_CASE(256)
    TFA_SFS_CASE(512)
    TFA_SFS_CASE(1024)
    TFA_SFS_CASE(2048)
    TFA_SFS_CASE(4096)
#undef TFA_SFS_CASE
    default: return hipErrorInvalidValue;
  }
}

template <int DIR>
static hipError_t launch_strided_fs_dir(const StridedFourStepArgs& a) {
  const int P = a.npass;
  long long N = 1;
  for (int i = 0; i < P; ++i) N *= a.len[i];
  const long long S = a.stride;
  const unsigned nmask = (unsigned)(N - 1);
  // pass 1 reads the input and writes the workspace; later non-final passes transform the
  // workspace in place (a workgroup writes exactly the addresses it read, after reading all of
  // them); the final pass reads the workspace and writes the output
  long long M_prev = N, K = 1;  // block length before this pass, product of earlier factors
  for (int i = 0; i < P; ++i) {
    const int L = a.len[i];
    const long long M = M_prev / L;
    const bool last = i == P - 1;
    SfsPass p{};
    p.S = S;
    p.lo_bits = a.lo_bits;
    p.nmask = nmask;
    p.scale = a.scale;
    hipError_t e;
    if (!last) {
      // blocks (o, k1..k_{i-1}) of M_prev*S floats; columns m*S + s over M*S
      p.blk = M_prev * S;
      p.tiles_per_block = M * S / sfs_tile(L);
      p.in_a = p.out_a = S;
      p.in_b = p.out_b = 0;
      p.qa_bits = kNoSplit;
      p.in_step = p.out_step = M * S;
      p.tw_mult = (unsigned)K;  // W_{M_prev}^x = W_N^(x*K)
      const float* src_re = i == 0 ? a.in_re : a.t_re;
      const float* src_im = i == 0 ? a.in_im : a.t_im;
      e = launch_sfs_pass<DIR>(L, src_re, src_im, a.t_re, a.t_im, a.tw[i], a, a.outer * K, true, p);
    } else {
      // columns col = (k1 + L1*k2 + ...)*S + s over K*S; block (o, k1..k_{P-1}) at row-major
      // index k1*(L2..L_{P-1}) + ... + k_{P-1} of LP*S floats each
      p.blk = N * S;
      p.tiles_per_block = K * S / sfs_tile(L);
      p.in_step = S;
      p.out_a = S;
      p.out_b = 0;
      p.out_step = K * S;
      if (P == 2) {
        p.qa_bits = kNoSplit;
        p.in_a = (long long)L * S;  // q = k1
        p.in_b = 0;
      } else {
        // q = k1 + L1*k2: block index k1*L2 + k2
        p.qa_bits = ilog2(a.len[0]);
        p.in_a = (long long)a.len[1] * L * S;
        p.in_b = (long long)L * S;
        p.out_b = (long long)a.len[0] * S;
      }
      p.tw_mult = 0;
      e = launch_sfs_pass<DIR>(L, a.t_re, a.t_im, a.out_re, a.out_im, a.tw[i], a, a.outer, false, p);
    }
    if (e != hipSuccess) return e;
    K *= L;
    M_prev = M;
  }
  return hipSuccess;
}

hipError_t launch_strided_fourstep(const StridedFourStepArgs& a) {
  if (a.npass < 2 || a.npass > 3 || a.outer < 1) return hipErrorInvalidValue;
  long long n = 1;
  for (int i = 0; i < a.npass; ++i) {
    if (a.len[i] < 64 || a.len[i] > 4096) return hipErrorInvalidValue;
    n *= a.len[i];
  }
  // stride 1: a contiguous axis (last pass staged through LDS); 4096-point last passes use the
  // split-plane exchange, which the staged pass does not have
  if (a.stride == 1 ? a.len[a.npass - 1] == 4096 : a.stride < strided_fs_min_stride(a.npass, n))
    return hipErrorInvalidValue;
  return a.dir < 0 ? launch_strided_fs_dir<-1>(a) : launch_strided_fs_dir<1>(a);
}

}  // namespace tfa
