// Dense / masked / variable-length MaxSim: host dispatch and the C entry points (the
// kernel template is in tms_dense_kernel.h).
//
// Reference semantics (src/flash_maxsim_v2.py:73-190, src/flash_maxsim_kernel.py:248-273,
// src/e2e_retrieval_quality.py:105-110): doc rows outside the document are -inf
// before the max, query rows past nq contribute 0, an empty document scores -inf.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "tms_dense_kernel.h"

namespace tms {

// Fixed-length documents (offsets null) or documents at offsets into T >= 1 rows, d in
// {32, 64, 96, 128} (tms_stream.hip).
int run_stream(const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd,
               const int64_t* offsets, int64_t T, int64_t pad_len, int dtype, float* out, hipStream_t st);
// Variable-length documents, d in {32, 64, 96, 128}, several query blocks (tms_stream.hip).
int run_varlen_batched(const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t T,
                       const int64_t* offsets, int64_t nd, int64_t B, int64_t pad_len, int dtype, float* out,
                       hipStream_t st, bool q32);
// Small batches (candidate reranking), documents split over several waves (tms_rerank.hip).
bool rerank_fits(int64_t B, int64_t tokens_per_doc);
int run_rerank(const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd, int64_t T,
               const int64_t* offsets, const uint8_t* mask, int64_t pad_len, int mode, int dtype, float* out,
               hipStream_t st);
// fp32 queries against fp16 / bf16 documents (tms_dense_q32.hip).
int run_dense_q32(DenseArgs a, int64_t nQ, int dtype, int mode, bool aligned, hipStream_t st);

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TMS_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return TMS_OK;
}

// Writes v into out[0..n).
__global__ void fill_kernel(float* out, int64_t n, float v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = v;
}

static int fill(float* out, int64_t n, float v, hipStream_t st) {
  if (n <= 0) return TMS_OK;
  int64_t grid = (n + 255) / 256;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)grid), dim3(256), 0, st, out, n, v);
  return check_launch("fill");
}

#ifndef TMS_DENSE_F32_TOKENS_PER_WAVE
#define TMS_DENSE_F32_TOKENS_PER_WAVE 768  // fp32 documents, d <= 128 (query in VGPRs)
#endif
#ifndef TMS_DENSE_F32_LDS_TOKENS_PER_WAVE
#define TMS_DENSE_F32_LDS_TOKENS_PER_WAVE 384  // fp32 documents, wider rows
#endif

// Documents per wave: short waves (about TMS_DENSE_TOKENS_PER_WAVE tokens, i.e. one
// document at typical ColBERT lengths) keep every CU's load pipeline full until the
// end of the launch and let the dispatcher balance ragged documents; the grid still
// spans at least two rounds of the chip's resident waves, and a wave never carries
// fewer tokens than it spends loading its query fragments. fp32 documents stream best
// with longer waves (measured per query, 192 / 384 / 768 tokens: C2 in fp32 14.3 / 13.7
// / 13.4 ms, C4 d = 768 in fp32 11.9 / 11.75 / 12.0 ms); 16-bit ones measured slower
// with 384 or 768.
static int pick_docs_per_wave(int64_t B, int64_t tokens_per_doc_hint, bool f32, int64_t d) {
  const int64_t tpw = !f32 ? TMS_DENSE_TOKENS_PER_WAVE
                           : (d <= 128 ? TMS_DENSE_F32_TOKENS_PER_WAVE : TMS_DENSE_F32_LDS_TOKENS_PER_WAVE);
  int64_t dpw = tokens_per_doc_hint > 0 ? tpw / tokens_per_doc_hint : 1;
  const int64_t min_waves = (int64_t)256 * 16 * 2;
  if (dpw > 1 && B / dpw < min_waves) dpw = B / min_waves;
  if (dpw < 1) dpw = 1;
  if (dpw > 64) dpw = 64;
  return (int)dpw;
}

static int dense_entry(const char* fn, const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B,
                       int64_t nd, int64_t total_tokens, const int64_t* offsets, const uint8_t* mask, int mode,
                       int dtype, float* out, void* stream, int64_t pad_len = 0) {
  const bool q32 = (dtype & TMS_QUERY_F32) != 0;  // fp32 queries (implied for fp32 documents)
  dtype &= ~TMS_QUERY_F32;
  if (dtype != TMS_DTYPE_F16 && dtype != TMS_DTYPE_BF16 && dtype != TMS_DTYPE_F32)
    return fail(TMS_ERR_UNSUPPORTED, "%s: unsupported dtype %d", fn, dtype);
  if (pad_len < 0) return fail(TMS_ERR_INVALID, "%s: negative pad_len %lld", fn, (long long)pad_len);
  if (nQ < 0 || nq < 0 || d < 0 || B < 0 || nd < 0 || total_tokens < 0)
    return fail(TMS_ERR_INVALID, "%s: negative size (nQ=%lld nq=%lld d=%lld B=%lld nd=%lld T=%lld)", fn, (long long)nQ,
                (long long)nq, (long long)d, (long long)B, (long long)nd, (long long)total_tokens);
  if (B == 0 || nQ == 0) return TMS_OK;
  if (!out) return fail(TMS_ERR_INVALID, "%s: out is NULL", fn);
  hipStream_t st = (hipStream_t)stream;
  if (nq == 0) return fill(out, nQ * B, 0.f, st);
  if (!Q) return fail(TMS_ERR_INVALID, "%s: Q is NULL", fn);
  if (mode == MODE_VARLEN && !offsets) return fail(TMS_ERR_INVALID, "%s: offsets is NULL", fn);
  if (mode == MODE_MASKED && nd > 0 && !mask) return fail(TMS_ERR_INVALID, "%s: mask is NULL", fn);
  const int64_t rows = (mode == MODE_VARLEN) ? total_tokens : B * nd;
  if (rows > 0 && d > 0 && !D) return fail(TMS_ERR_INVALID, "%s: D is NULL", fn);
  if (d > kMaxDim) return fail(TMS_ERR_UNSUPPORTED, "%s: d=%lld > %d is not supported", fn, (long long)d, kMaxDim);
  if (nq > (int64_t)1 << 24 || nQ > (int64_t)1 << 20 || nQ * ((nq + 31) / 32) > ((int64_t)1 << 30))
    return fail(TMS_ERR_UNSUPPORTED, "%s: too many query tokens", fn);

  DenseArgs a;
  memset(&a, 0, sizeof(a));
  a.Q = (const uint8_t*)Q;
  a.D = (const uint8_t*)D;
  a.offsets = offsets;
  a.mask = mask;
  a.out = out;
  a.B = B;
  a.nd = nd;
  a.total_tokens = total_tokens;
  a.nq = (int32_t)nq;
  a.nbq = (int32_t)((nq + 31) / 32);
  a.d = (int32_t)d;
  a.nchunk = (int32_t)((d + 7) / 8);
  a.nstep = (int32_t)((d + 31) / 32);
  a.nkg = (int32_t)((a.nstep + 3) / 4);
  if (a.nkg < 1) a.nkg = 1;
  int64_t hint = (mode == MODE_VARLEN) ? (B > 0 ? total_tokens / B : 0) : nd;
  a.docs_per_wave = pick_docs_per_wave(B, hint, dtype == TMS_DTYPE_F32, d);
  a.pad_len = pad_len;
  a.mask4 = (nd % 4 == 0 && ((uintptr_t)mask & 3) == 0) ? 1 : 0;
  const bool aligned = (d % 8 == 0) && (((uintptr_t)Q & 15) == 0) && (((uintptr_t)D & 15) == 0);
  const bool qreg = aligned && d > 0 && d <= 128 && d % 32 == 0;
  // fp32 documents or fp32 queries, several query blocks: the shared-tile kernel (one pass
  // for up to 16 blocks; three or two MFMAs per product) instead of one pass per one or
  // two blocks
  if ((dtype == TMS_DTYPE_F32 || q32) && mode != MODE_MASKED && qreg && a.nbq <= 2 && nQ * a.nbq > 2)
    return run_varlen_batched(Q, nQ, nq, d, D, mode == MODE_VARLEN ? total_tokens : B * nd,
                              mode == MODE_VARLEN ? offsets : nullptr, nd, B, pad_len, dtype, out, st,
                              dtype != TMS_DTYPE_F32);
  if (dtype == TMS_DTYPE_F32) return run_dense<TMS_DTYPE_F32, TMS_DTYPE_F32>(a, nQ, mode, aligned, st);
  if (q32) return run_dense_q32(a, nQ, dtype, mode, aligned, st);
  // a few thousand documents or fewer against one or two query blocks: each document split
  // over up to four waves, so that small calls still fill the chip
  if (qreg && nQ * a.nbq <= 3 && rerank_fits(B, hint))
    return run_rerank(Q, nQ, nq, d, D, B, nd, total_tokens, offsets, mask, pad_len, mode, dtype, out, st);
  if (mode == MODE_FIXED && qreg) return run_stream(Q, nQ, nq, d, D, B, nd, nullptr, 0, 0, dtype, out, st);
  if (mode == MODE_VARLEN && qreg && a.nbq <= 4 && nQ * a.nbq >= 4)  // one pass for up to 32 blocks
    return run_varlen_batched(Q, nQ, nq, d, D, total_tokens, offsets, 0, B, pad_len, dtype, out, st, false);
  // variable-length documents against one or two query blocks per pass: the stream kernel,
  // whose walk reads each wave's document bounds from its lanes (no rows: the general kernel)
  if (mode == MODE_VARLEN && qreg && total_tokens > 0)
    return run_stream(Q, nQ, nq, d, D, B, 0, offsets, total_tokens, pad_len, dtype, out, st);
  if (dtype == TMS_DTYPE_F16) return run_dense<TMS_DTYPE_F16, TMS_DTYPE_F16>(a, nQ, mode, aligned, st);
  return run_dense<TMS_DTYPE_BF16, TMS_DTYPE_BF16>(a, nQ, mode, aligned, st);
}

}  // namespace tms

extern "C" {

int tms_version(void) { return 100; }

const char* tms_last_error(void) { return tms::g_err; }

int tms_maxsim_dense(const void* Q, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd, int dtype, float* out,
                     void* stream) {
  return tms::dense_entry("tms_maxsim_dense", Q, 1, nq, d, D, B, nd, 0, nullptr, nullptr, tms::MODE_FIXED, dtype, out,
                          stream);
}

int tms_maxsim_masked(const void* Q, int64_t nq, int64_t d, const void* D, const uint8_t* mask, int64_t B, int64_t nd,
                      int dtype, float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_masked", Q, 1, nq, d, D, B, nd, 0, nullptr, mask, tms::MODE_MASKED, dtype, out,
                          stream);
}

int tms_maxsim_varlen(const void* Q, int64_t nq, int64_t d, const void* D_flat, int64_t total_tokens,
                      const int64_t* offsets, int64_t B, int dtype, float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_varlen", Q, 1, nq, d, D_flat, B, 0, total_tokens, offsets, nullptr,
                          tms::MODE_VARLEN, dtype, out, stream);
}

int tms_maxsim_varlen_padded(const void* Q, int64_t nq, int64_t d, const void* D_flat, int64_t total_tokens,
                             const int64_t* offsets, int64_t B, int64_t pad_len, int dtype, float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_varlen_padded", Q, 1, nq, d, D_flat, B, 0, total_tokens, offsets, nullptr,
                          tms::MODE_VARLEN, dtype, out, stream, pad_len);
}

int tms_maxsim_varlen_batched(const void* Qs, int64_t nQ, int64_t nq, int64_t d, const void* D_flat,
                              int64_t total_tokens, const int64_t* offsets, int64_t B, int64_t pad_len, int dtype,
                              float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_varlen_batched", Qs, nQ, nq, d, D_flat, B, 0, total_tokens, offsets, nullptr,
                          tms::MODE_VARLEN, dtype, out, stream, pad_len);
}

int tms_maxsim_dense_batched(const void* Qs, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd,
                             int dtype, float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_dense_batched", Qs, nQ, nq, d, D, B, nd, 0, nullptr, nullptr, tms::MODE_FIXED,
                          dtype, out, stream);
}

}  // extern "C"
