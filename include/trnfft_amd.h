/*
 * trnfft_amd.h — C ABI of the MI355X (gfx950) FFT backend for trnfft.
 *
 * Plain C: raw device pointers, sizes and an opaque stream handle; no torch types.  Data is in
 * trnfft's split layout (ComplexTensor, trnfft/complex.py:16-33): two contiguous row-major
 * fp32 planes, re and im, batch rows of length n.  All entry points return TFA_OK (0) or a
 * negative status; tfa_last_error() gives the calling thread's message for the last failure.
 *
 * Ownership: the caller owns every input, output and workspace buffer (device memory, e.g. from
 * the PyTorch caching allocator).  A plan owns its device tables (twiddles, Bluestein chirp and
 * filter spectrum, DFT matrix) and is immutable after creation, so tfa_execute* may be called
 * concurrently on one plan from several threads/streams.  A plan is bound to the device that was
 * current at creation.
 */
#ifndef TRNFFT_AMD_H
#define TRNFFT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tfa_plan tfa_plan;
typedef void* tfa_stream; /* hipStream_t; NULL = the null stream */

/* Status codes (the Python layer maps them to exceptions). */
#define TFA_OK 0
#define TFA_ERR_INVALID (-1)     /* bad argument                      -> ValueError          */
#define TFA_ERR_UNSUPPORTED (-2) /* size or kind not implemented      -> NotImplementedError */
#define TFA_ERR_HIP (-3)         /* HIP runtime / launch failure      -> RuntimeError        */

/* Plan kinds. */
#define TFA_KIND_C2C 0       /* power-of-two n (Stockham in LDS; four-step above 16384)     */
#define TFA_KIND_BLUESTEIN 1 /* any n >= 2, chirp-z over a power-of-two m >= 2n-1            */
#define TFA_KIND_DFT_GEMM 2  /* n <= 256, X = x @ W on the matrix cores                      */
#define TFA_KIND_STFT 3      /* framed, windowed onesided/twosided transform of real signals */
#define TFA_KIND_FFT2 4      /* 2-D transform over the last two axes (n = last, n2 = second to last) */
#define TFA_KIND_REAL 5      /* real rows: forward r2c (n real -> n/2+1 bins), inverse c2r; power-of-two 4 <= n <= 32768 */

/* STFT flags. */
#define TFA_STFT_CENTER 1     /* reflect-pad n_fft/2 on both sides (pad_mode="reflect") */
#define TFA_STFT_NORMALIZED 2 /* scale by 1/sqrt(n_fft)                                 */
#define TFA_STFT_ONESIDED 4   /* keep bins 0..n_fft/2                                   */
/* Spectra stored (batch, n_frames, n_bins) row-major instead of (batch, n_bins, n_frames).  Without
 * it the planes are trnfft's result layout: its stft wraps the transposed frame spectra in a
 * ComplexTensor, whose constructor makes them contiguous (trnfft/api.py:357-365,
 * trnfft/complex.py:29-33).  With it they are in the memory order of torch.stft's
 * (..., freq, time) result (no reference counterpart).  Applies to the forward output, the
 * inverse input and the backward's gradient input. */
#define TFA_STFT_FRAMES_MAJOR 8

typedef struct tfa_plan_desc {
  int32_t kind;    /* TFA_KIND_* */
  int32_t inverse; /* 0: forward, sign -1, unscaled; 1: inverse, sign +1, scaled 1/n */
  int64_t n;       /* transform length (STFT: n_fft) */
  int64_t hop;     /* STFT only: hop_length */
  int32_t flags;   /* STFT only: TFA_STFT_* */
  int32_t reserved;
  int64_t n2;      /* FFT2 only: length of the second-to-last axis */
} tfa_plan_desc;

/*
 * Create a plan.  Replaces the reference's per-call plan lookup plus table construction:
 * trnfft/plan.py:34-46 (create_plan: algorithm choice, Bluestein m = 1 << (2n-2).bit_length()),
 * trnfft/fft_core.py:86-88 (radix-2 twiddles), :1316-1345 (Bluestein chirp, with the same
 * fp32 angle expression sign*pi*k*k/n, and filter h), :239-243 (DFT matrix).
 */
int tfa_plan_create(tfa_plan** out, const tfa_plan_desc* desc);

/* Release a plan and its device tables (trnfft/plan.py:49-50 clear_plan_cache drops them). */
void tfa_plan_destroy(tfa_plan* plan);

/* Device workspace (bytes) tfa_execute needs for `batch` rows; 0 when none. */
int tfa_plan_workspace_size(const tfa_plan* plan, int64_t batch, size_t* bytes);

/* Padded length m of a Bluestein plan (n for the other kinds). */
int64_t tfa_plan_padded_n(const tfa_plan* plan);

/*
 * Batched 1-D transform along the last axis: out[b, k] = sum_j in[b, j] W^(j k) (x 1/n when
 * inverse).  in_im may be NULL for real input (imaginary part zero, trnfft/complex.py:27-28).
 * Out-of-place, or in place with out_* == in_*.  Replaces trnfft/fft_core.py:22-50 (fft_core),
 * which dispatches to _cooley_tukey (:53-117, power-of-two n), _bluestein (:1285-1376, other n)
 * and, for TFA_KIND_DFT_GEMM plans, _fft_via_gemm (:221-251).
 * TFA_KIND_FFT2 plans: `batch` arrays of (n2, n) each, transformed over both axes (x 1/(n n2)
 * when inverse), power-of-two 16 <= n <= 4096 and 16 <= n2 <= 4096 (two HBM passes), or
 * n * n2 <= 16384 with both axes >= 4 (>= 8 at 8192, >= 16 at 16384; whole images in LDS, one
 * pass); output must not alias the input; replaces trnfft/api.py:105-139 (fft2 -> fftn over
 * (-2, -1)).
 * TFA_KIND_REAL plans, forward (replaces trnfft/api.py:38-46, rfft): in_re = (batch, n) real
 * rows, in_im must be NULL, out_re/out_im = (batch, n/2+1) bins.  Inverse (replaces
 * trnfft/api.py:49-68, irfft with its default n = 2*(bins-1)): in_re/in_im = (batch, n/2+1)
 * bins, out_re = (batch, n) real rows scaled 1/n, out_im unused (may be NULL); the imaginary
 * parts of bins 0 and n/2 are ignored, as the reference's real part of the Hermitian-completed
 * inverse ignores them.  The real rows (input of the forward, output of the inverse) must be
 * 8-byte aligned; out-of-place only.
 */
int tfa_execute(const tfa_plan* plan, int64_t batch, const float* in_re, const float* in_im,
                float* out_re, float* out_im, void* workspace, tfa_stream stream);

/*
 * tfa_execute without a workspace argument and without any device allocation: the scratch the
 * four-step (n > 16384) and split-Bluestein kernels need comes from a static device array of
 * 64 MiB per GPU, part of the library's code object and held until the process ends.  No
 * counterpart in the reference; it is for callers that cannot allocate device memory (code under
 * HIP-graph capture, serving loops, harnesses that forbid hipMalloc).  A call whose scratch
 * (tfa_plan_workspace_size) exceeds 64 MiB fails with TFA_ERR_INVALID; plans that need no scratch
 * run exactly as tfa_execute.  Every call on one GPU shares that GPU's scratch: eager calls are
 * ordered on the device by the library (each waits, on its stream, for an event the previous
 * eager call recorded), but calls made while the stream is capturing a HIP graph are not, so
 * graph replays that overlap other noalloc calls on the same GPU race.
 */
int tfa_execute_noalloc(const tfa_plan* plan, int64_t batch, const float* in_re, const float* in_im,
                        float* out_re, float* out_im, tfa_stream stream);

/*
 * Batched 1-D transform along a strided axis, in place allowed: data viewed as (outer, n, stride)
 * row-major, each of the outer*stride columns transformed along its n elements (element stride
 * `stride`).  TFA_KIND_C2C plans with n <= 4096, or TFA_KIND_BLUESTEIN plans with n <= 2048
 * (padded length m <= 4096).  Replaces the transpose-copy + contiguous FFT + transpose-back of
 * trnfft/api.py:496-516 (_fft_along_dim) used by fft2/fftn/ifftn.
 */
int tfa_execute_strided(const tfa_plan* plan, int64_t outer, int64_t stride, const float* in_re,
                        const float* in_im, float* out_re, float* out_im, tfa_stream stream);

/*
 * tfa_execute_strided extended to power-of-two TFA_KIND_C2C axes 4096 < n <= 2^24 with
 * stride >= 4 (>= 8 from n = 2^21): two strided passes (three from 2^21) through `workspace`,
 * whose size tfa_strided_workspace_size reports (2 * 4 * outer * n * stride bytes for such axes,
 * else 0).  n = 4096 with stride >= 16 also takes two passes (faster than the single pass there).
 * In place allowed (out_* == in_*); the workspace must not overlap the data.  Every other
 * plan/stride goes to tfa_execute_strided (workspace unused).  outer = 0 is a no-op on both entry
 * points (the size query then reports 0 bytes).  Replaces the same transposes of
 * trnfft/api.py:496-516 for long axes.
 */
int tfa_strided_workspace_size(const tfa_plan* plan, int64_t outer, int64_t stride, size_t* bytes);
int tfa_execute_strided_ws(const tfa_plan* plan, int64_t outer, int64_t stride, const float* in_re,
                           const float* in_im, float* out_re, float* out_im, void* workspace, tfa_stream stream);

/*
 * Short-time Fourier transform of `batch` real signals of `num_samples` samples each.  Frames
 * of n_fft samples every hop, after reflect padding when TFA_STFT_CENTER; each frame is
 * multiplied by window (device pointer, n_fft floats, already centre-padded to n_fft) and
 * transformed; output planes are (batch, n_bins, n_frames) row-major, or (batch, n_frames,
 * n_bins) with TFA_STFT_FRAMES_MAJOR, with n_bins = n_fft/2+1 when TFA_STFT_ONESIDED else n_fft.  Replaces trnfft/api.py:291-365 (stft).  n_fft: a power
 * of two in [16, 4096], or any other n_fft from 9 up to 2731 (onesided) or 2048 (two-sided),
 * forward only: each frame then goes through the reference's Bluestein chain
 * (trnfft/fft_core.py:1285-1376), convolved at the shortest power of two or 3 * 2^k that holds
 * n_fft + n_bins - 1 points.
 */
int tfa_stft_frames(const tfa_plan* plan, int64_t num_samples, int64_t* n_frames);
int tfa_stft_execute(const tfa_plan* plan, int64_t batch, int64_t num_samples, const float* signal,
                     const float* window, float* out_re, float* out_im, tfa_stream stream);

/*
 * Complex GEMM on split planes, C = A @ B (b_trans = 0) or C = A @ B^T (b_trans = 1), plus an
 * optional complex bias broadcast over rows (bias_re/bias_im NULL for none).  A is (m, k) with
 * row stride lda; B is (k, n) with row stride ldb, or (n, k) when b_trans; C is (m, n) with row
 * stride ldc.  Replaces trnfft/nki/dispatch.py:74-84 (complex_gemm) and :91-102
 * (complex_linear: y = x @ W^T with W (out, in)), whose kernels are :121-200 and :267-345, and
 * the bias add of trnfft/nn.py:46-48.
 */
int tfa_complex_gemm(int64_t m, int64_t n, int64_t k, const float* a_re, const float* a_im,
                     int64_t lda, const float* b_re, const float* b_im, int64_t ldb, int32_t b_trans,
                     const float* bias_re, const float* bias_im, float* c_re, float* c_im,
                     int64_t ldc, tfa_stream stream);

/*
 * Inverse STFT (TFA_KIND_STFT plan created with inverse = 1; n = n_fft, hop, flags CENTER /
 * NORMALIZED / ONESIDED, FRAMES_MAJOR optional): spec_re/spec_im (batch, n_bins, n_frames), or
 * (batch, n_frames, n_bins) with FRAMES_MAJOR, with n_bins = n/2+1 when ONESIDED else n, -> out
 * (batch, out_len), out_len from tfa_istft_length (length < 0: the default length).
 * Hermitian completion (onesided) or the real part of each frame's inverse transform (two-sided,
 * power-of-two n only), inverse transform, window, overlap-add, division by the window-square
 * envelope where it exceeds 1e-8 (the raw overlap-add elsewhere), centre trim and zero fill to
 * `length` in one kernel.  Replaces trnfft/api.py:368-470 (istft), whose per-frame loops
 * (:438-452) and window-sum masking (:450-452) it fuses.
 */
int tfa_istft_length(const tfa_plan* plan, int64_t n_frames, int64_t length, int64_t* out_len);
int tfa_istft_execute(const tfa_plan* plan, int64_t batch, int64_t n_frames, const float* spec_re,
                      const float* spec_im, const float* window, float* out, int64_t length, tfa_stream stream);

/*
 * Gradient of the onesided forward STFT with respect to its padded signal: grad_re/grad_im
 * (batch, n/2+1, n_frames), or (batch, n_frames, n/2+1) when the plan has FRAMES_MAJOR, the
 * gradient of tfa_stft_execute's output planes, -> grad_padded
 * (batch, padded_len), padded_len = num_samples + 2*(n/2) when CENTER else num_samples, n_frames
 * = 1 + (padded_len - n)/hop.  Per frame the adjoint of the r2c transform (interior bins halved,
 * Hermitian-completed inverse transform, unscaled; 1/sqrt(n) when NORMALIZED), times the window,
 * overlap-added; samples no frame covers get zero.  n_fft that is not a power of two: per frame
 * the adjoint of the Bluestein chain the forward kernel runs (conj(chirp) times the gradient,
 * convolved with chirp[|s|], times conj(chirp)).  Undoing the centre padding (the reflected edges
 * folded back) is left to the caller.  Runs on the forward STFT plan of the call being
 * differentiated (ONESIDED required); a hop whose recomputed halo frames would fill the kernel's
 * frame tile returns TFA_ERR_UNSUPPORTED.  Replaces the backward that torch autograd derives for
 * trnfft/api.py:310-349 (pad, frame index, window multiply, per-frame transform): a
 * gather-transpose of the gradient, an inverse transform per frame and an index_add/fold
 * overlap-add.
 */
int tfa_stft_backward_execute(const tfa_plan* plan, int64_t batch, int64_t n_frames, const float* grad_re,
                              const float* grad_im, const float* window, float* grad_padded, int64_t padded_len,
                              tfa_stream stream);

/* Operand ops of tfa_complex_gemm_ex (BLAS-style, plus conjugation without transpose). */
#define TFA_OP_N 0 /* op(X) = X          */
#define TFA_OP_T 1 /* op(X) = X^T        */
#define TFA_OP_C 2 /* op(X) = conj(X)^T  */
#define TFA_OP_R 3 /* op(X) = conj(X)    */

/*
 * General complex GEMM on split planes: C = alpha * op(A) @ op(B) + bias, op(A) (m, k), op(B)
 * (k, n).  A is stored (m, k), or (k, m) for TFA_OP_T/TFA_OP_C, with row stride lda; B is stored
 * (k, n), or (n, k) for TFA_OP_T/TFA_OP_C, with row stride ldb.  These are the adjoint products
 * of trnfft/nki/autograd.py:92-155 (_ComplexGEMMFn.backward dA = dC B^H, dB = A^H dC;
 * _ComplexLinearFn.backward dX = dY conj(W), dW = dY^T conj(X)), which the reference runs as
 * eight real torch matmuls; here each is one launch.
 */
int tfa_complex_gemm_ex(int64_t m, int64_t n, int64_t k, const float* a_re, const float* a_im, int64_t lda,
                        int32_t a_op, const float* b_re, const float* b_im, int64_t ldb, int32_t b_op, float alpha,
                        const float* bias_re, const float* bias_im, float* c_re, float* c_im, int64_t ldc,
                        tfa_stream stream);

/*
 * Strided-batched form of tfa_complex_gemm_ex: for b in [0, batch),
 *   C_b = alpha * op(A_b) @ op(B_b) + bias,  X_b = X + b * stride_x (floats, both planes).
 * A stride of 0 shares that operand across the batch (broadcast); C's stride must separate the
 * output matrices.  Replaces the batched and broadcast torch.matmul products of
 * trnfft/complex.py:142-150 (complex_matmul / ComplexTensor.__matmul__: four real matmuls of
 * (..., m, k) @ (..., k, n) operands), one launch for all four products of every matrix pair.
 */
int tfa_complex_gemm_batched(int64_t batch, int64_t m, int64_t n, int64_t k, const float* a_re, const float* a_im,
                             int64_t lda, int64_t stride_a, int32_t a_op, const float* b_re, const float* b_im,
                             int64_t ldb, int64_t stride_b, int32_t b_op, float alpha, const float* bias_re,
                             const float* bias_im, float* c_re, float* c_im, int64_t ldc, int64_t stride_c,
                             tfa_stream stream);

/* Thread-local message describing the last failure on this thread ("" if none). */
const char* tfa_last_error(void);

/* ABI version, (major << 16) | minor. */
int32_t tfa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TRNFFT_AMD_H */
