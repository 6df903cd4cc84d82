/*
 * tilemaxsim C ABI -- fused MaxSim / PQ-ADC scoring on one MI355X (gfx950).
 *
 * Every entry point takes device pointers and plain sizes, enqueues its kernels on
 * `stream` (a hipStream_t passed as void*; NULL = the legacy default stream) and
 * returns without synchronising. Nothing here allocates device memory.
 * Arguments are validated before any HIP call; a non-zero return is one of the
 * TMS_ERR_* codes and tms_last_error() gives the message (per host thread).
 *
 * Layouts are row-major and dense: Q (nq, d); D (B, nd, d); D_flat (T, d);
 * offsets (B + 1) int64; mask (B, nd) bytes (non-zero = real token);
 * codebook (M, K, dsub); codes (B, nd, M) uint8; lut (nq, M, K) fp32; out (B) fp32.
 * Element type of Q / D / codebook is given by `dtype` (TMS_DTYPE_*).
 *
 * Scores follow the reference: score[b] = sum_i max_j <Q[i], D[b, j]> with fp32
 * accumulation; a document with no (unmasked) token scores -inf; nq == 0 gives 0.
 */
#ifndef TILEMAXSIM_H
#define TILEMAXSIM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TMS_OK 0
#define TMS_ERR_INVALID 1     /* bad argument (shape, pointer, offsets) */
#define TMS_ERR_UNSUPPORTED 2 /* valid but not implemented (dtype, size limit) */
#define TMS_ERR_HIP 3         /* the HIP runtime reported an error */

#define TMS_DTYPE_F16 0
#define TMS_DTYPE_BF16 1
/* fp32 embeddings: taken by the dense entry points (tms_maxsim_*) and by
 * tms_pq_build_lut. Each element is split into two bf16 terms (hi + lo) on the fly and
 * every product is formed from three bf16 products, so its relative error is at most
 * about 3 * 2^-16 (the reference computes fp32 inputs with TF32 tl.dot, about 2^-10). */
#define TMS_DTYPE_F32 2
/* OR-ed into the dtype of a dense entry point (tms_maxsim_*), of tms_pq_build_lut or of
 * tms_pq_score: Q is fp32 while the documents / codebook are the fp16 or bf16 `dtype`.
 * The query is not rounded to 16 bits: each element is split into hi + lo terms of the
 * document type (fp16: after a per-token power-of-two scale, which the max commutes
 * with) and a product takes two MFMAs, relative error about 2^-17 (bf16) or 2^-21
 * (fp16) per element; the reference computes fp32 x 16-bit products with TF32 tl.dot
 * (2^-11). Redundant with TMS_DTYPE_F32 documents, whose queries are fp32 already. */
#define TMS_QUERY_F32 0x100
/* OR-ed into the dtype of tms_pq_score / tms_pq_score_batched: `codes` points to int16
 * (TMS_CODES_I16) or int32 (TMS_CODES_I32) codes, read at that width, instead of uint8.
 * Codes at or beyond K (or negative) are invalid input and are clamped into the table. */
#define TMS_CODES_I16 0x200
#define TMS_CODES_I32 0x400

/* Library version (major * 10000 + minor * 100 + patch). */
int tms_version(void);

/* Message for the last non-zero status returned on this host thread. */
const char* tms_last_error(void);

/*
 * Small-batch dispatch limit of the dense entry points (tms_maxsim_dense, _masked,
 * _varlen, _varlen_padded, and the batched ones with at most three 32-token query
 * blocks in all): a call whose documents span at most `tiles` 16-token tiles
 * (B * ceil(mean tokens per document / 16)), with fp16 / bf16 embeddings and d in
 * {32, 64, 96, 128}, takes the small-batch kernel, which splits each document over up
 * to four waves so that a few hundred candidates still fill the chip; larger calls
 * stream whole documents per wave. Default 16384 tiles (measured on MI355X: the
 * small-batch kernel takes 0.6-0.7x the time up to about 500 documents and about the
 * same at 1,000-2,000). The same limit (B * ceil(mean tokens per indexed document /
 * 16)) lets tms_maxsim_residual split candidate documents over two or four waves while
 * the call stays within three waves per SIMD (256 candidates: 16 -> 8 us). Sets the
 * limit when tiles >= 0 and returns the previous one (tiles < 0 only returns it).
 * Process-wide. Both forms give the same bits. No reference counterpart (a tuning
 * control, and what tests use to run both forms on the same inputs).
 */
int64_t tms_set_rerank_limit(int64_t tiles);

/*
 * Dense fixed-length MaxSim, every d (the d <= 128 kernel and the d-tiled kernel).
 * Replaces flash_maxsim_v2_multiquery (src/flash_maxsim_v2.py:227-289) and its two
 * kernels _flash_maxsim_v2_multiquery_kernel (:73-130) and
 * _flash_maxsim_v2_mq_dimtile_kernel (:133-190); also serves flash_maxsim_v2
 * (:193-224), flash_maxsim_batch (src/flash_maxsim_kernel.py:200-245) and
 * flash_maxsim_single (:167-197), which compute the same scores.
 */
int tms_maxsim_dense(const void* Q, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd, int dtype,
                     float* out, void* stream);

/*
 * Dense MaxSim with a per-token validity mask: masked tokens are -inf before the max.
 * Replaces the masked PyTorch scorer pytorch_maxsim_score(Q, D, D_mask)
 * (src/e2e_retrieval_quality.py:105-110).
 */
int tms_maxsim_masked(const void* Q, int64_t nq, int64_t d, const void* D, const uint8_t* mask, int64_t B,
                      int64_t nd, int dtype, float* out, void* stream);

/*
 * Variable-length MaxSim over a flat token buffer: document b is
 * D_flat[offsets[b] : offsets[b+1]]. Offsets must be non-decreasing within
 * [0, total_tokens]; a document whose offsets violate that scores NaN.
 * Replaces flash_maxsim_multi_doc (src/flash_maxsim_kernel.py:248-273).
 */
int tms_maxsim_varlen(const void* Q, int64_t nq, int64_t d, const void* D_flat, int64_t total_tokens,
                      const int64_t* offsets, int64_t B, int dtype, float* out, void* stream);

/*
 * Variable-length MaxSim with the zero-padding semantics of the reference's PLAID
 * drop-in: each document is scored as if zero-padded to pad_len tokens, so a document
 * shorter than pad_len also sees dot products of 0 (its per-query-token max is at
 * least 0, and an empty one scores 0). Nothing is padded in memory.
 * Replaces flashmaxsim_score_packed (src/plaid_integration_benchmark.py:154-183), which
 * builds the padded (B, max_len, d) tensor, zeroes its padding and runs the dense kernel.
 */
int tms_maxsim_varlen_padded(const void* Q, int64_t nq, int64_t d, const void* D_flat, int64_t total_tokens,
                             const int64_t* offsets, int64_t B, int64_t pad_len, int dtype, float* out, void* stream);

/*
 * Batched-query dense MaxSim: nQ queries of nq tokens each (Qs is (nQ, nq, d)) scored
 * against the same documents in one pass over D; out is (nQ, B), row-major.
 * Replaces nQ calls of flash_maxsim_v2_multiquery (src/flash_maxsim_v2.py:227-289).
 */
int tms_maxsim_dense_batched(const void* Qs, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B,
                             int64_t nd, int dtype, float* out, void* stream);

/*
 * Batched-query MaxSim over variable-length documents: nQ queries of nq tokens (Qs is
 * (nQ, nq, d)) against the documents of tms_maxsim_varlen / tms_maxsim_varlen_padded
 * (pad_len 0: empty documents score -inf; pad_len > 0: the zero-padding semantics);
 * out is (nQ, B), row-major. With d in {32, 64, 96, 128}, 16-byte aligned Qs and
 * D_flat and at most 128 tokens per query, up to 32 query blocks of 32 tokens share
 * each pass over D_flat.
 * Replaces nQ calls of flash_maxsim_multi_doc (src/flash_maxsim_kernel.py:248-273) or of
 * flashmaxsim_score_packed (src/plaid_integration_benchmark.py:154-183) over the same
 * documents.
 */
int tms_maxsim_varlen_batched(const void* Qs, int64_t nQ, int64_t nq, int64_t d, const void* D_flat,
                              int64_t total_tokens, const int64_t* offsets, int64_t B, int64_t pad_len, int dtype,
                              float* out, void* stream);

/*
 * PQ distance table lut[q, m, k] = sum_j Q[q, m*dsub + j] * codebook[m, k, j] (fp32;
 * fp16, bf16 or fp32 Q and codebook of one dtype, or with TMS_QUERY_F32 an fp32 Q
 * against an fp16 / bf16 codebook, used unrounded). Replaces
 * TileMaxSimPQ.build_distance_table (src/flash_pqsim_kernel.py:190-211) and
 * _build_distance_table_kernel (:31-67).
 */
int tms_pq_build_lut(const void* Q, int64_t nq, const void* codebook, int64_t M, int64_t K, int64_t dsub, int dtype,
                     float* lut, void* stream);

/*
 * PQ MaxSim by table gather: out[b] = sum_q max_t sum_m lut[q, m, codes[b, t, m]].
 * Replaces _flash_pqsim_batched_score_kernel (src/flash_pqsim_kernel.py:127-173) plus the
 * host q-sum (:250), i.e. the scoring half of TileMaxSimPQ.score_batch (:213-252).
 */
int tms_pq_score_lut(const float* lut, int64_t nq, int64_t M, int64_t K, const uint8_t* codes, int64_t B, int64_t nd,
                     float* out, void* stream);

/*
 * tms_pq_score_lut for codes of code_bytes = 1, 2 or 4 bytes (uint8, int16, int32), read
 * at their own width, and any K (the reference scores int32 codes with no K limit,
 * src/flash_pqsim_kernel.py:219,233,161-165). Tables of M * K <= 16384 entries per query
 * token are gathered from LDS slices of query tokens; larger ones from slices tiled over
 * m as well, with per-token partial sums in registers (documents of up to 4096 tokens);
 * tables with K > 16384, or longer documents, straight from memory. Codes at or beyond
 * K are clamped into the table.
 */
int tms_pq_score_lut_ex(const float* lut, int64_t nq, int64_t M, int64_t K, const void* codes, int code_bytes,
                        int64_t B, int64_t nd, float* out, void* stream);

/*
 * PQ MaxSim by codebook gather: each document token is rebuilt from the codebook in
 * registers (never in HBM) and scored on MFMA; same scores as tms_pq_score_lut up to
 * fp32 summation order. Replaces TileMaxSimPQ.score_batch (src/flash_pqsim_kernel.py:
 * 213-252) as a whole. Shapes: d = M * dsub in {32, 64, 96, 128}, dsub in {2, 4, 8, 16,
 * 32}, M a multiple of 4, a codebook of d * K 16-bit elements that fits the device's LDS
 * (K <= 640 at d = 128 on gfx950's 160 KiB), 16-byte aligned Q, codebook and codes,
 * nd * M * code bytes < 2^31, and an fp16 or bf16 codebook. dtype flags: TMS_QUERY_F32
 * (fp32 Q, uint8 codes), TMS_CODES_I16 / TMS_CODES_I32. Other shapes and fp32 codebooks
 * return TMS_ERR_UNSUPPORTED before any HIP call (score them with tms_pq_build_lut +
 * tms_pq_score_lut_ex).
 */
int tms_pq_score(const void* Q, int64_t nq, const void* codebook, int64_t M, int64_t K, int64_t dsub, int dtype,
                 const uint8_t* codes, int64_t B, int64_t nd, float* out, void* stream);

/*
 * Batched-query PQ scoring: nQ queries of nq tokens (Qs is (nQ, nq, M*dsub)) against the
 * same codes; out is (nQ, B), row-major. Shapes and dtype flags as tms_pq_score; with
 * uint8 codes, a query of the codebook's type, a codebook of at most 64 KiB and at most
 * 128 tokens per query, each 16-token tile is decoded once per pass (codes gathered
 * through the codebook in LDS) and shared by up to 32 query blocks of 32 tokens; other
 * inputs are scored one query at a time. Replaces nQ calls of TileMaxSimPQ.score_batch
 * (src/flash_pqsim_kernel.py:213-252) over the same codes.
 */
int tms_pq_score_batched(const void* Qs, int64_t nQ, int64_t nq, const void* codebook, int64_t M, int64_t K,
                         int64_t dsub, int dtype, const uint8_t* codes, int64_t B, int64_t nd, float* out,
                         void* stream);

/*
 * Row-wise top-k of an fp32 score matrix (nrows, n): values (nrows, k) descending with
 * int64 indices; equal values come out in ascending index order and NaN ranks above
 * +inf. Needs tms_topk_workspace_size(nrows, n, k) bytes of device workspace (0 when a
 * row fits one 4096-element chunk). k <= 1024, n < 2^32, nrows <= 65535 per call.
 * Replaces torch.topk(scores, k) in the reference's retrieval step
 * (src/cycle3_experiments.py:215).
 */
int tms_topk(const float* scores, int64_t nrows, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
             float* out_values, int64_t* out_indices, void* stream);

/* Device workspace in bytes that tms_topk needs for these sizes (0 if none or invalid). */
int64_t tms_topk_workspace_size(int64_t nrows, int64_t n, int64_t k);

/*
 * tms_topk without a workspace argument: allocates nothing and takes no caller memory
 * beyond its inputs and outputs. No counterpart in the reference; it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The intermediate keys live in a fixed 32 MiB device
 * array of the library (TMS_TOPK_SCRATCH_BYTES; one copy per GPU, held until the process
 * ends). The array sits in a code object of its own, with no kernels: under HIP's
 * deferred module loading (the ROCm default) a GPU reserves it at the first
 * tms_topk_noalloc call there, and processes that only call tms_topk never do. That first
 * call on each device loads the array and looks up its address, so it must not run under
 * stream capture: make one call eagerly before capturing tms_topk_noalloc into a graph
 * (later calls launch kernels only and capture like tms_topk). The calling thread's
 * current device must be the one that holds the pointers and the stream. Sizes whose
 * tms_topk_workspace_size() exceeds the array return TMS_ERR_UNSUPPORTED (split the rows
 * over several calls). Every call on one GPU shares its array: calls that overlap on
 * one GPU (different streams, or host threads, with no ordering between them) race, and
 * must be serialised by the caller. Results equal tms_topk's bit for bit.
 */
#define TMS_TOPK_SCRATCH_BYTES (32LL << 20)
int tms_topk_noalloc(const float* scores, int64_t nrows, int64_t n, int64_t k, float* out_values,
                     int64_t* out_indices, void* stream);

/*
 * MaxSim of one query against B <= 1024 fixed-length documents and their top-k, in one
 * launch: the small-batch scoring kernel writes the B scores, and the workgroup that
 * finishes last selects the top k of them (values descending, ties to the lower index,
 * the same bits as tms_maxsim_dense followed by tms_topk). fp16 / bf16, 1..64 query
 * tokens, d in {32, 64, 96, 128}, 16-byte aligned Q and D, 1 <= k <= B; other shapes
 * return TMS_ERR_UNSUPPORTED (score, then tms_topk). `counter` is a device block of
 * TMS_MAXSIM_TOPK_COUNTER_WORDS 32-bit words (the workgroups' tickets, taken in two levels
 * on large grids, each counter on its own 64-byte line) that must hold 0 before the first
 * call; each call leaves it 0 again. Calls that share a counter must not overlap (calls on
 * one stream never do). Replaces the reference's
 * scoring call followed by torch.topk (src/cycle3_experiments.py:215) for the serving
 * shapes of the reference's reranking flow (src/e2e_retrieval_quality.py:267-291).
 */
#define TMS_MAXSIM_TOPK_COUNTER_WORDS 144
int tms_maxsim_topk(const void* Q, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd, int dtype, int64_t k,
                    float* scores, float* out_values, int64_t* out_indices, uint32_t* counter, void* stream);

/*
 * Residual-compressed documents: the ColBERTv2 codec (ResidualCodec in
 * colbert/indexing/codecs/residual.py) of colbert-ai 0.2.22, the ColBERT release the
 * reference's PLAID drop-in is written against (src/plaid_integration_benchmark.py:23).
 * Token t of the index is a centroid id codes[t] (int32) and a residual row of
 * d * nbits / 8 bytes at residuals + t * d * nbits / 8: for each dimension, bits
 * 0 .. nbits-1 of its bucket index (least significant first), dimensions in order,
 * packed from the most significant bit of each byte. It decodes to
 *   v = fp16(centroids[code] + bucket_weights[bucket]),  x = fp16(v / fp16(|v|)).
 * centroids (ncent, d) and bucket_weights (2^nbits) are fp16; nbits is 1, 2 or 4;
 * d is 32, 64, 96 or 128. Centroid ids outside [0, ncent) are clamped.
 */

/*
 * Decompress T tokens into out (T, d) fp16 (16-byte aligned).
 * Replaces ResidualCodec.decompress (GPU path) of colbert-ai 0.2.22, which PLAID runs on
 * candidate documents before the scorer the reference replaces
 * (src/plaid_integration_benchmark.py:154-183).
 */
int tms_residual_decompress(const int32_t* codes, const uint8_t* residuals, int64_t T, const void* centroids,
                            int64_t ncent, int64_t d, const void* bucket_weights, int nbits, void* out, void* stream);

/*
 * MaxSim of one fp16 query Q (nq, d) against residual-compressed documents, decoded in
 * registers: no decompressed copy is written. Document p < ndocs is index rows
 * [offsets[p], offsets[p+1]) of total_tokens; out[b] scores document pids[b] (or b when
 * pids is NULL, then B <= ndocs). pad_len > 0 gives the zero-padding semantics of
 * tms_maxsim_varlen_padded; 0 gives plain MaxSim (an empty document scores -inf). An
 * invalid pid or offsets scores NaN. Each token's dot products are scaled by
 * 1 / fp16(|v|) before the max, so scores equal MaxSim over the decompressed tokens up
 * to their fp16 rounding.
 * Replaces, in the reference's PLAID path, ColBERT's decompression of the candidates
 * followed by flashmaxsim_score_packed (src/plaid_integration_benchmark.py:154-183).
 */
int tms_maxsim_residual(const void* Q, int64_t nq, int64_t d, const void* centroids, int64_t ncent,
                        const void* bucket_weights, int nbits, const int32_t* codes, const uint8_t* residuals,
                        int64_t total_tokens, const int64_t* offsets, int64_t ndocs, const int64_t* pids, int64_t B,
                        int64_t pad_len, float* out, void* stream);

/*
 * Batched-query MaxSim over residual-compressed documents: nQ fp16 queries of nq tokens
 * (Qs is (nQ, nq, d)) against the same documents, with the arguments and semantics of
 * tms_maxsim_residual; out is (nQ, B), row-major. Each 16-token tile is decoded once
 * per pass and shared by up to 32 query blocks of 32 tokens, and the decoded tokens are
 * rounded to fp16 as the codec rounds them (x = fp16(v * (1 / fp16(|v|)))).
 * Replaces nQ rounds of ColBERT's decompression followed by flashmaxsim_score_packed
 * (src/plaid_integration_benchmark.py:154-183) when the queries share their candidates,
 * as in exhaustive scoring of a compressed collection.
 */
int tms_maxsim_residual_batched(const void* Qs, int64_t nQ, int64_t nq, int64_t d, const void* centroids,
                                int64_t ncent, const void* bucket_weights, int nbits, const int32_t* codes,
                                const uint8_t* residuals, int64_t total_tokens, const int64_t* offsets, int64_t ndocs,
                                const int64_t* pids, int64_t B, int64_t pad_len, float* out, void* stream);

/*
 * Measurement helper, not part of the scoring path and with no counterpart in the
 * reference: reads `bytes` (a multiple of 8 KiB) of `buf` once with a read-only
 * streaming kernel and writes one XOR word per thread to `sink`
 * (TMS_READ_PROBE_SINK_WORDS words). `bench.py --config readprobe` times it over a
 * C2-sized buffer: the read rate any streaming kernel on this part can reach.
 */
#define TMS_READ_PROBE_SINK_WORDS 524288
int tms_read_probe(const void* buf, int64_t bytes, uint32_t* sink, int64_t sink_words, void* stream);

/*
 * Measurement helper, not part of the scoring path and with no counterpart in the
 * reference: times 16 x 4096 x 16 ds_read_b128 wave-instructions per CU (256 workgroups
 * of 16 waves, 128 KiB of LDS each) for one lane -> address pattern (0: conflict-free,
 * 1: the PQ kernel's codebook gather, 2: every lane group on one bank group, 3: four
 * lanes of each 16-lane group per bank group); patterns 4 to 7 are 0 to 3 at the PQ
 * kernel's occupancy and footprint (512 workgroups of 8 waves, two per CU, 64 KiB of
 * LDS each); patterns 8 and 9 are 5 and 4 with two v_mfma_f32_16x16x32_f16 per gathered
 * fragment on random fp16 data (the PQ kernel's matrix work beside its gathers);
 * patterns 10 and 11 (at the shape of 0 to 3) are conflict-free and two-way
 * respectively under the part's pass rule (four passes of 16 lanes, the lanes that share
 * lane bit 5 and the parity of lane bits 2-4), and the other way round if the passes were
 * 16 consecutive lanes. Writes each wave's elapsed s_memtime count to `cycles`
 * (TMS_LDS_PROBE_WAVES words) and one word per thread to `sink` (64 x
 * TMS_LDS_PROBE_WAVES words). `bench.py --config ldsprobe` runs the twelve patterns.
 */
#define TMS_LDS_PROBE_WAVES 4096
int tms_lds_probe(int pattern, int64_t* cycles, int64_t cycle_words, uint32_t* sink, int64_t sink_words,
                  void* stream);

/*
 * Measurement helper, not part of the scoring path and with no counterpart in the
 * reference: 512 workgroups of 4 waves (2 waves per SIMD) issue nothing but
 * v_mfma_f32_16x16x32_f16 on operands read once from `ops` (512 16-byte fp16
 * fragments), eight accumulators per wave, and write one word per thread to `sink`
 * (TMS_MFMA_PROBE_SINK_WORDS words). `*flops` receives the launch's MFMA FLOPs.
 * `bench.py --config mfmaprobe` times it on random operands: the sustained MFMA rate
 * of this part at the clock it holds under that load.
 */
#define TMS_MFMA_PROBE_SINK_WORDS 131072
int tms_mfma_probe(const void* ops, float* sink, int64_t sink_words, int64_t* flops, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TILEMAXSIM_H */
