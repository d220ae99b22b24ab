/* nxg_linear.h -- C ABI of the MI355X (gfx950) int8 linear-layer engine for NexteraBERT.
 *
 * The engine replaces the int8 path of NexteraBERT.cpp: per-token activation
 * quantization, the W8A8 GEMM over load-time-expanded weights with int32
 * accumulation, and the dequant/scale (+residual) epilogue, over the packed,
 * unpadded rows of a mixed-length batch. Results are the reference's bit for bit:
 * the same int32 block sums and the same fp32 outputs.
 *
 * Conventions
 *   - Plain pointers and sizes only. Device pointers are HIP device memory on the
 *     current device; host pointers are ordinary memory. `stream` is a hipStream_t
 *     (NULL: the default stream); device work is ordered by it and the calls return
 *     without waiting for it.
 *   - Every int-returning call returns NXG_OK (0) or an NXG_E* code, the reference C
 *     API's convention (0 ok, 1 bad input, 2 allocation, 3 compute;
 *     src/nexterabert.cpp:1874-1899). nxg_last_error() gives the reason.
 *   - One host thread per engine object at a time, like a nextera_context
 *     (src/nexterabert.cpp:342-344).
 *
 * Buffers on the device
 *   quantized activations of T rows x n_in inputs ("qact"):
 *     q   int8, nxg_qact_q_bytes(T, n_in) bytes, in MFMA fragment tiles: byte (t, k) at
 *           ((t/16)*KS + k/64)*1024 + ((t%16) + 16*((k%64)/16))*16 + k%16,
 *         KS = ceil(n_in/64); values are the reference's u8 minus ACT_OFF; padding is 0.
 *     sx  float, nxg_qact_sx_bytes(T, n_in) bytes, in the reference's layout
 *           [token/4][block][token%4] (src/nexterabert.cpp:368-375), padded to 16 rows.
 *   outputs and residuals: float [T][n_out], row-major (the (n_out, T) ggml tensor).
 *   Every device buffer above, and the fp32 rows the quantizers and producers read, must be
 *   16-byte aligned (hipMalloc gives 256); a call given another refuses it with NXG_EINVAL.
 */
#ifndef NXG_LINEAR_H
#define NXG_LINEAR_H

#include <stddef.h>
#include <stdint.h>

#if defined(NXG_BUILD)
#  define NXG_API __attribute__((visibility("default")))
#else
#  define NXG_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define NXG_OK      0
#define NXG_EINVAL  1   /* bad input */
#define NXG_ENOMEM  2   /* allocation failed */
#define NXG_EDEVICE 3   /* HIP error, missing or wrong GPU */

#define NXG_BLOCK 256   /* inputs per scale block: I8_BLOCK, src/nexterabert.cpp:254 */

/* ggml block types the load-time expansion decodes (ggml's type numbering, as stored in GGUF). */
enum nxg_type {
    NXG_TYPE_F32  = 0,
    NXG_TYPE_F16  = 1,
    NXG_TYPE_Q4_0 = 2,
    NXG_TYPE_Q4_1 = 3,
    NXG_TYPE_Q5_0 = 6,
    NXG_TYPE_Q5_1 = 7,
    NXG_TYPE_Q8_0 = 8,
    NXG_TYPE_Q2_K = 10,
    NXG_TYPE_Q3_K = 11,
    NXG_TYPE_Q4_K = 12,
    NXG_TYPE_Q5_K = 13,
    NXG_TYPE_Q6_K = 14,
    NXG_TYPE_BF16 = 30
};

/* Reason for the last failed call on this thread ("" if none). */
NXG_API const char * nxg_last_error(void);

/* ---------------------------------------------------------------------------
 * Host side: load-time weight expansion
 * ------------------------------------------------------------------------- */

/* Would the reference run this weight on its int8 GEMM? Replaces the placement rule
 * of nextera_load, src/nexterabert.cpp:1658-1667: use_int8, 2-D, a quantized block type,
 * not an embedding matrix, ne0 % 32 == 0 and ne1 % 4 == 0. Returns 1 or 0. */
NXG_API int32_t nxg_weight_is_int8(const char * name, int32_t n_dims, int32_t type,
                                   int64_t ne0, int64_t ne1, int32_t use_int8);

/* Bytes of one row of n_in values of `type` in a GGUF file (ggml_row_size); 0 if unsupported. */
NXG_API size_t nxg_row_bytes(int32_t type, int64_t n_in);

/* Decode rows of a GGUF tensor to f32 (ggml's to_float for `type`). out: n_rows * n_in floats. */
NXG_API int32_t nxg_dequantize_rows(int32_t type, const void * data, int64_t n_in, int64_t n_rows, float * out);

/* build_i8_weight, src/nexterabert.cpp:1010-1049: dequantize each of the n_out rows of
 * `data` (ggml `type`, n_in values per row) and re-quantize every block of 256 inputs
 * to s8 with lround(x * 127/amax).
 *   w      out: int8  [n_out][n_in]
 *   scale  out: float [n_blk][n_out], amax / 127
 *   off    out: int32 [n_blk][n_out], -act_off * sum of the block's s8 values (may be NULL;
 *               act_off is ACT_MAX + 1: 128 on VNNI builds of the reference, 64 on AVX2 ones)
 * n_threads <= 0: all hardware threads. */
NXG_API int32_t nxg_expand_weight(int32_t type, const void * data, int32_t n_in, int32_t n_out,
                                  int32_t act_off, int32_t n_threads,
                                  int8_t * w, float * scale, int32_t * off);

/* Encodes n_rows rows of n_in f32 values as Q8_0, Q5_0, Q4_K or Q6_K GGUF blocks into
 * nxg_row_bytes(type, n_in) * n_rows bytes at `out`. For synthetic weight files; the
 * reference's own quantizer is ggml's (tools/quantize.cpp:201-213), whose search for
 * K-quant scales this one-pass encoder does not reproduce. */
NXG_API int32_t nxg_quantize_weight(int32_t type, const float * x, int64_t n_in, int64_t n_rows, void * out);

/* ---------------------------------------------------------------------------
 * Device side
 * ------------------------------------------------------------------------- */

/* Checks that the current HIP device is a gfx950 GPU. Called by every device entry
 * point on first use; returns NXG_EDEVICE otherwise. */
NXG_API int32_t nxg_init(void);

/* Sizes of the qact buffers for T rows of n_in inputs (0 if n_in is not a positive
 * multiple of 32 or T < 0). */
NXG_API size_t nxg_qact_q_bytes(int32_t T, int32_t n_in);
NXG_API size_t nxg_qact_sx_bytes(int32_t T, int32_t n_in);

/* quantize_row on every row (src/nexterabert.cpp:378-403; op_copy, :453-461).
 *   x        device float [T][n_in]
 *   act_max  127 (VNNI builds of the reference) or 63 (AVX2-only builds), src/nexterabert.cpp:53-70
 *   q, sx    device qact buffers (sizes above); fully written, padding included. */
NXG_API int32_t nxg_quantize_rows(const float * x, int32_t T, int32_t n_in, int32_t act_max,
                                  int8_t * q, float * sx, void * stream);

/* op_relu_sqr with an int8 consumer (src/nexterabert.cpp:484-505, quantized by
 * for_rows, :414-438; chosen by row_op(..., int8_only(c_proj)), :1287-1288): every
 * element becomes r*r with r = x > 0 ? x : 0 (a NaN gives 0), then quantize_row as
 * nxg_quantize_rows. Same arguments. */
NXG_API int32_t nxg_quantize_rows_relu2(const float * x, int32_t T, int32_t n_in, int32_t act_max,
                                        int8_t * q, float * sx, void * stream);

/* op_rms_norm with an int8 consumer (src/nexterabert.cpp:463-482, quantized by for_rows,
 * :414-438; chosen by rms_norm(..., int8_only(...)), e.g. :1285): each row becomes
 * (x * inv) * gain with inv = 1 / sqrt(dot / n_in + eps), dot = dot_f32(x, x) in the
 * reference's AVX2 accumulation order (:124-149), then quantize_row as nxg_quantize_rows.
 *   x     device float [T][n_in], 16-byte aligned
 *   gain  device float [n_in] (the norm's weight), 16-byte aligned;  eps  the model's rms_norm_epsilon */
NXG_API int32_t nxg_rmsnorm_quantize_rows(const float * x, const float * gain, float eps, int32_t T, int32_t n_in,
                                          int32_t act_max, int8_t * q, float * sx, void * stream);

/* The mixers' producers with an int8 consumer: each computes its rows as the
 * reference's AVX2 build does (n_in % 32 == 0, so its scalar tails never run) and
 * quantizes them as nxg_quantize_rows (for_rows' quantize branch, :414-438). All
 * arrays are device arrays, rows of n_in floats. Unlike nxg_linear_i8, the packed
 * layout here is on the device: cu_offsets (and cu_blocks) hold n_seqs + 1 int32,
 * strictly increasing from 0 (the reference's layout::start plus total, :231-244,
 * :1341-1354); other offsets give unspecified rows but never an out-of-bounds access. */

/* op_gate (src/nexterabert.cpp:507-522), the input of every gated mixer's c_proj
 * (gated_out, :1208-1213): out = sigmoid(g) * y, sigmoid(g) = 1 / (1 + exp(0 - g))
 * with exp as exp256 computes it (:81-100, :119-122). g, y: [T][n_in]. */
NXG_API int32_t nxg_gate_quantize_rows(const float * g, const float * y, int32_t T, int32_t n_in, int32_t act_max,
                                       int8_t * q, float * sx, void * stream);

/* op_dwconv (src/nexterabert.cpp:524-543), SnowLily's input of ltc_conv.out_proj
 * (:1233-1236): out[t] = r[t] (or 0 if r is null), then for j = 0 .. k-1 with
 * t + j - k/2 inside t's document, out[t] = fma(taps[j], x[t + j - k/2], out[t]).
 * x, r: [T][n_in]; taps: [k][n_in] (the layout conv_params hands over, :1152-1159). */
NXG_API int32_t nxg_dwconv_quantize_rows(const float * x, const float * r, const float * taps, int32_t k,
                                         const int32_t * cu_offsets, int32_t n_seqs, int32_t T, int32_t n_in,
                                         int32_t act_max, int8_t * q, float * sx, void * stream);

/* op_lily_state (src/nexterabert.cpp:545-578), the input of SnowLily's c_proj
 * (:1239-1243): acc = 0, then for the taps j with t + j - k/2 inside t's document,
 * acc = fma(taps[j], a[t+j-k/2] * x[t+j-k/2], acc); out[t] = acc * b[t].
 * a, x, b: [T][n_in]; taps: [k][n_in]. */
NXG_API int32_t nxg_lily_state_quantize_rows(const float * a, const float * x, const float * b, const float * taps,
                                             int32_t k, const int32_t * cu_offsets, int32_t n_seqs, int32_t T,
                                             int32_t n_in, int32_t act_max, int8_t * q, float * sx, void * stream);

/* op_block_mean (src/nexterabert.cpp:638-659), the input of HRA's c_q / c_k / c_v
 * (:1253-1256): block row b of document d is the mean of its (up to block) tokens,
 * out = 0, out = fma(h, g, out) per token in order (out + h without g), then
 * out * (1 / n). h, g (nullable): [T][n_in] tokens; cu_blocks: the block rows'
 * layout, ceil(len_d / block) rows per document, n_blocks = cu_blocks[n_seqs];
 * q, sx: a qact of n_blocks rows. */
NXG_API int32_t nxg_block_mean_quantize_rows(const float * h, const float * g, const int32_t * cu_offsets,
                                             const int32_t * cu_blocks, int32_t n_seqs, int32_t T, int32_t n_blocks,
                                             int32_t block, int32_t n_in, int32_t act_max, int8_t * q, float * sx,
                                             void * stream);

/* op_attention with head_dim 64 (src/nexterabert.cpp:704-852): grouped-query attention
 * inside each document of a packed layout, with the reference's AVX2 arithmetic (the
 * scores' 8-lane FMA chains and their two summation trees, softmax_exp with exp256 and the
 * C library's expf for the last n % 8 keys, the value sums in key order).
 *   q         device float [T][n_head * 64], row-major (after qk_prep)
 *   k, v      device float [n_kv_head][T][64], head-major
 *   cu_offsets, n_seqs  the packed layout on the device (as the producers take it)
 *   scale     device float [n_seqs]: the per-document scale (nxg_attention_scales)
 *   half      -1: every key of the document; >= 0: the band |i - j| <= half (swa)
 *   max_keys  an upper bound of keys per query (a query with more gets NaN outputs); with
 *             n_head / n_kv_head not dividing 16, at most 16384
 *   out       device float [T][n_head * 64] */
NXG_API int32_t nxg_attention(const float * q, const float * k, const float * v, const int32_t * cu_offsets,
                              int32_t n_seqs, const float * scale, int32_t T, int32_t n_head, int32_t n_kv_head,
                              int32_t half, int32_t max_keys, float * out, void * stream);

/* op_attention (src/nexterabert.cpp:785-852) as nxg_attention, with a device workspace for
 * launches whose scores do not fit in LDS (more than ~2,400 keys per query with
 * n_head / n_kv_head dividing 16), or fit with room for one workgroup per CU (more than ~1,200
 * keys), or for two in a launch of more than 4 x the CUs' workgroups (e.g. 2 x 1,024 keys):
 * each score is computed once and kept in the workspace for the softmax and the values,
 * instead of kept in LDS or recomputed in each of three passes; the outputs are the same bits.
 * The workspace holds one slot of 16 * max_keys floats per resident workgroup; a smaller one
 * (at least one slot) runs fewer workgroups at a time, and none (NULL, 0) the LDS kernel where
 * its scores fit, else the recomputing kernel. Other launches ignore it.
 * Calls that share a workspace must not overlap.
 *   workspace        device memory, 4-byte aligned, or NULL
 *   workspace_bytes  its size (nxg_attention_workspace_bytes gives the size for every slot) */
NXG_API int32_t nxg_attention_ws(const float * q, const float * k, const float * v, const int32_t * cu_offsets,
                                 int32_t n_seqs, const float * scale, int32_t T, int32_t n_head, int32_t n_kv_head,
                                 int32_t half, int32_t max_keys, float * out, void * workspace,
                                 int64_t workspace_bytes, void * stream);

/* nxg_attention_ws without a caller's workspace and without allocating: no counterpart in
 * the reference; for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The workspace is a static
 * device array of NXG_NOALLOC_SCRATCH_BYTES in the library's code object, one per GPU, held
 * until the process ends -- by every process that loads the library, on each GPU it uses,
 * whether or not it calls this entry point; the call uses as many of its slots (16 * max_keys floats each) as fit, and
 * refuses (NXG_EINVAL) a max_keys whose single slot would not fit (more than 1,048,576 keys) where the
 * scores do not fit in LDS either.
 * Same arguments and results as nxg_attention. Calls that overlap on one GPU race (they
 * share the array); calls in one stream, or synchronized, do not. */
#define NXG_NOALLOC_SCRATCH_BYTES (64u << 20)
NXG_API int32_t nxg_attention_noalloc(const float * q, const float * k, const float * v, const int32_t * cu_offsets,
                                      int32_t n_seqs, const float * scale, int32_t T, int32_t n_head,
                                      int32_t n_kv_head, int32_t half, int32_t max_keys, float * out, void * stream);

/* Sizing for nxg_attention_ws (no counterpart in the reference, whose op_attention keeps a
 * document's scores in host memory): the workspace it uses for these sizes: 0 when the launch does not need one,
 * else one slot per resident workgroup (a negative NXG_E* code for invalid sizes). */
NXG_API int64_t nxg_attention_workspace_bytes(int32_t T, int32_t n_head, int32_t n_kv_head, int32_t max_keys);

/* op_qk_prep (src/nexterabert.cpp:590-632): the separable DyT (beta * tanh(alpha * x), with
 * tanh256's arithmetic) then RoPE at each row's position in its document:
 *   x          device float [T][n_head * head_dim]
 *   alpha, beta device float [head_dim] (the q_norm / k_norm parameters)
 *   cos_t, sin_t device float [n_pos][head_dim / 2] (nxg_rope_table), n_pos > the longest document
 *   out        device float, row-major [T][n_head * head_dim] (head_major 0, queries) or
 *              head-major [n_head][T][head_dim] (head_major 1, keys) */
NXG_API int32_t nxg_qk_prep(const float * x, const float * alpha, const float * beta, const float * cos_t,
                            const float * sin_t, int32_t n_pos, const int32_t * cu_offsets, int32_t n_seqs,
                            int32_t T, int32_t n_head, int32_t head_dim, int32_t head_major, float * out,
                            void * stream);

/* op_head_major (src/nexterabert.cpp:620-632): device [T][n_head * head_dim] -> [n_head][T][head_dim]. */
NXG_API int32_t nxg_head_major(const float * x, int32_t T, int32_t n_head, int32_t head_dim, float * out,
                               void * stream);

/* The three ops builder::attention applies to one layer's projections (src/nexterabert.cpp:
 * 1186-1188) in one launch, each element as by the separate calls: nxg_qk_prep of the
 * queries q [T][n_head * head_dim] (q_alpha / q_beta, row-major into q_out), nxg_qk_prep of
 * the keys k [T][n_kv_head * head_dim] (k_alpha / k_beta, head-major into k_out) and
 * nxg_head_major of the values v into v_out. */
NXG_API int32_t nxg_qkv_prep(const float * q, const float * k, const float * v, const float * q_alpha,
                             const float * q_beta, const float * k_alpha, const float * k_beta, const float * cos_t,
                             const float * sin_t, int32_t n_pos, const int32_t * cu_offsets, int32_t n_seqs,
                             int32_t T, int32_t n_head, int32_t n_kv_head, int32_t head_dim, float * q_out,
                             float * k_out, float * v_out, void * stream);

/* op_dwconv writing fp32 rows (src/nexterabert.cpp:524-543, row_op(..., false): HRA's qkv_conv
 * and c_o, :1252, :1265): out = r (or 0 with r null), then out = fma(taps[j], x[t + j - k/2], out)
 * for the taps j whose row lies in t's document, in order of j.
 *   x, r       device float [T][C] (C % 4 == 0; 16-byte aligned)
 *   taps       device float [k][C] (the loader's per-tap rows, :1703-1710)
 *   cu_offsets device int32 [n_seqs + 1]
 *   out        device float [T][C] */
NXG_API int32_t nxg_dwconv_rows(const float * x, const float * r, const float * taps, int32_t k,
                                const int32_t * cu_offsets, int32_t n_seqs, int32_t T, int32_t C, float * out,
                                void * stream);

/* op_upsample_add (src/nexterabert.cpp:675-690): out[t] = yb[cu_blocks[d] + (t - cu_offsets[d]) / block]
 * + r[t] for row t of document d.
 *   yb   device float [n_blocks][C] (one row per block of `block` tokens, per document)
 *   r    device float [T][C];  cu_offsets, cu_blocks device int32 [n_seqs + 1];  out [T][C] */
NXG_API int32_t nxg_upsample_add(const float * yb, const float * r, const int32_t * cu_offsets,
                                 const int32_t * cu_blocks, int32_t n_seqs, int32_t T, int32_t n_blocks,
                                 int32_t block, int32_t C, float * out, void * stream);

/* The encoder's input rows (src/nexterabert.cpp:1271-1272): ggml_get_rows of the embedding,
 * plus the segment embedding's row (ggml_add) when type_table is given.
 *   table       device float [n_vocab][C] (a block-quantized file table decoded once)
 *   ids         device int32 [T] (checked on the host: an id outside the table is clamped)
 *   type_table  device float [n_types][C] or null;  types  device int32 [T]
 *   out         device float [T][C] */
NXG_API int32_t nxg_embed_rows(const float * table, int32_t n_vocab, const int32_t * ids, const float * type_table,
                               int32_t n_types, const int32_t * types, int32_t T, int32_t C, float * out,
                               void * stream);

/* ggml_norm then ggml_mul by w and ggml_add of b (the encoder's out_norm, src/nexterabert.cpp:
 * 1290-1291; the heads' transform, :1296-1297, has no b). ggml (v0.9.9) is not in the reference's
 * tree: mean and variance are taken in double as its CPU op publishes them, in a fixed lane order.
 *   x  device float [T][C];  w, b  device float [C] or null;  out  device float [T][C] */
NXG_API int32_t nxg_layer_norm(const float * x, const float * w, const float * b, float eps, int32_t T, int32_t C,
                               float * out, void * stream);

/* nextera_encode's pooled output (src/nexterabert.cpp:1913-1925) and op_doc_mean (:659-672): the
 * sum of each document's rows in row order, times 1 / n, or with normalize != 0 times
 * 1 / sqrt(dot_f32(p, p)) (0 for a zero vector; C % 32 == 0).
 *   x  device float [T][C];  cu_offsets device int32 [n_seqs + 1];  out  device float [n_seqs][C] */
NXG_API int32_t nxg_doc_mean(const float * x, const int32_t * cu_offsets, int32_t n_seqs, int32_t T, int32_t C,
                             int32_t normalize, float * out, void * stream);

/* build_rope (src/nexterabert.cpp:1322-1338) on the host with the same C library calls:
 * cos / sin of t * (1 / base^(2i / head_dim)) for t < n_pos, i < head_dim / 2.
 *   cos_out, sin_out  host float [n_pos][head_dim / 2] */
NXG_API int32_t nxg_rope_table(int32_t n_pos, float base, int32_t head_dim, float * cos_out, float * sin_out);

/* The per-document scales op_attention uses (src/nexterabert.cpp:1196-1201, :1174-1181),
 * on the host with the C library's logf: base = 1 / sqrt(head_dim); mode 0 (ssmax "none"
 * or an swa layer): base; 1 ("ssmax"): base * (s * ln n); 2 ("sssmax"): base *
 * (s * ln n + ssmax_base + max(b, 0)); n = max(document length, 1).
 *   cu_offsets  host int32, n_seqs + 1;  out  host float [n_seqs] */
NXG_API int32_t nxg_attention_scales(const int32_t * cu_offsets, int32_t n_seqs, int32_t head_dim, int32_t mode,
                                     float s, float b, float ssmax_base, float * out);

/* The qact buffers in the reference's own format (src/nexterabert.cpp:368-375):
 *   u8  device uint8 [T][n_in], the reference's u8 values (q + act_max + 1)
 *   sx_ref device float, ((T+3)/4)*n_blk*4 floats, [token/4][block][token%4] */
NXG_API int32_t nxg_qact_export(const int8_t * q, const float * sx, int32_t T, int32_t n_in, int32_t act_max,
                                uint8_t * u8, float * sx_ref, void * stream);

/* An expanded weight on the device, re-laid out once into MFMA fragment tiles. */
typedef struct nxg_weight nxg_weight;

/* Uploads an expanded weight (host w [n_out][n_in], scale [n_blk][n_out] as written by
 * nxg_expand_weight; the i8_weight of src/nexterabert.cpp:256-261 without `off`, which
 * the signed activations make unnecessary). n_in: positive multiple of 32; n_out >= 1.
 * Blocks until the upload is complete. */
NXG_API int32_t nxg_weight_create(const int8_t * w, const float * scale, int32_t n_in, int32_t n_out,
                                  nxg_weight ** out);
NXG_API void    nxg_weight_destroy(nxg_weight * w);
NXG_API int32_t nxg_weight_n_in(const nxg_weight * w);
NXG_API int32_t nxg_weight_n_out(const nxg_weight * w);
/* Bytes of device memory the weight holds. */
NXG_API size_t  nxg_weight_device_bytes(const nxg_weight * w);

/* op_linear_i8, src/nexterabert.cpp:969-1007 (registered by builder::linear, :1121-1138):
 *   out[t][r] = residual[t][r] + f,  f = fma((float) s_B * sx[t,B], scale[B][r], f) over B
 * ascending, s_B the exact int32 sum of block B. Rows are the packed batch: cu_offsets
 * (host int32, n_seqs + 1 entries, cu_offsets[0] = 0, strictly increasing -- empty
 * sequences are refused as in src/nexterabert.cpp:1345-1347) gives T = cu_offsets[n_seqs].
 *   q, sx     qact of the T rows (from nxg_quantize_rows)
 *   residual  device float [T][n_out] or NULL
 *   out       device float [T][n_out] */
NXG_API int32_t nxg_linear_i8(const nxg_weight * w, const int8_t * q, const float * sx,
                              const int32_t * cu_offsets, int32_t n_seqs,
                              const float * residual, float * out, void * stream);

/* The same for T rows given directly. */
NXG_API int32_t nxg_linear_i8_rows(const nxg_weight * w, const int8_t * q, const float * sx, int32_t T,
                                   const float * residual, float * out, void * stream);

/* nxg_linear_i8_rows for projections that share an input, fused along n_out into one weight
 * (rows and per-block scales concatenated): columns [c_k, c_k + cols[k]) of the product,
 * c_k = cols[0] + ... + cols[k-1], go to outs[k], a dense device float [T][cols[k]] array,
 * so one launch replaces n_seg calls of builder::linear (src/nexterabert.cpp:1121-1138) on
 * the same qact. Each column is computed exactly as by nxg_linear_i8_rows. No residual;
 * n_in % 256 == 0; 1 <= n_seg <= 4; every boundary c_k (k > 0) a multiple of 64 and every
 * cols[k] a multiple of 4, summing to n_out; outs[k] 16-byte aligned. */
NXG_API int32_t nxg_linear_i8_rows_split(const nxg_weight * w, const int8_t * q, const float * sx, int32_t T,
                                         int32_t n_seg, const int32_t * cols, float * const * outs, void * stream);

/* The MLP's c_fc -> relu^2 -> int8 in one pass (src/nexterabert.cpp:1286-1288: linear
 * of c_fc, then op_relu_sqr quantized for the int8 c_proj): the fp32 linear output f of
 * nxg_linear_i8 (no residual) is never written; q_out, sx_out receive exactly what
 * nxg_quantize_rows_relu2 would produce from it, a qact of T rows by n_out inputs
 * (sizes nxg_qact_q_bytes(T, n_out), nxg_qact_sx_bytes(T, n_out)), padding included.
 * Needs n_in % 256 == 0 and n_out % 32 == 0 (NXG_EINVAL otherwise); act_max is that of
 * the consumer, 127 or 63. */
NXG_API int32_t nxg_linear_i8_relu2_q8(const nxg_weight * w, const int8_t * q, const float * sx,
                                       const int32_t * cu_offsets, int32_t n_seqs, int32_t act_max,
                                       int8_t * q_out, float * sx_out, void * stream);

/* The same for T rows given directly. */
NXG_API int32_t nxg_linear_i8_relu2_q8_rows(const nxg_weight * w, const int8_t * q, const float * sx, int32_t T,
                                            int32_t act_max, int8_t * q_out, float * sx_out, void * stream);

/* The same from fp32 rows, as op_linear_i8 takes them (src/nexterabert.cpp:969-1007: the
 * input rows quantized by quantize_row, :378-403, then the int8 GEMM): x device float
 * [T][n_in], 16-byte aligned; act_max that of the model (the input's quantization and the
 * output's), 127 or 63. The result equals nxg_quantize_rows(x) followed by
 * nxg_linear_i8_relu2_q8_rows, bit for bit. Where the row-tile kernel runs (n_in 256 or 1024)
 * with at least 4 tiles of 64 rows by 256 outputs per workgroup (two workgroups per compute
 * unit: 16,384 rows of 2,304 outputs on 256 CUs), each row tile is quantized inside the GEMM
 * and the int8 input never goes to memory; otherwise q_ws, sx_ws (a qact of T rows by n_in, nxg_qact_q_bytes(T, n_in) and
 * nxg_qact_sx_bytes(T, n_in) bytes) receive nxg_quantize_rows(x) first. The workspace is
 * required in either case (whether the fused kernel runs depends on the device's CU count). */
NXG_API int32_t nxg_linear_f32_relu2_q8_rows(const nxg_weight * w, const float * x, int32_t T, int32_t act_max,
                                             int8_t * q_ws, float * sx_ws, int8_t * q_out, float * sx_out,
                                             void * stream);

/* The same over a packed batch: T = cu_offsets[n_seqs] (host int32, as nxg_linear_i8). */
NXG_API int32_t nxg_linear_f32_relu2_q8(const nxg_weight * w, const float * x, const int32_t * cu_offsets,
                                        int32_t n_seqs, int32_t act_max, int8_t * q_ws, float * sx_ws,
                                        int8_t * q_out, float * sx_out, void * stream);

/* The int32 block sums s_B of the same GEMM: sums device int32 [n_blk][T][n_out],
 * equal to the reference's sum_i w8*u8 + off (src/nexterabert.cpp:892-916). For tests. */
NXG_API int32_t nxg_linear_i8_block_sums(const nxg_weight * w, const int8_t * q, int32_t T,
                                         int32_t * sums, void * stream);

/* Diagnostic, no counterpart in the reference (whose op_linear_i8 has one kernel): the
 * kernel a GEMM of T rows, n_in inputs and n_out outputs launches, as the profiler names
 * its template instance (e.g. "gemm_k256<true>"), for a device of `cus` compute units
 * (cus <= 0: the current device, which must be a gfx950 GPU). flags: NXG_GEMM_RESIDUAL
 * (nxg_linear_i8 with a residual), NXG_GEMM_RELU2 (nxg_linear_i8_relu2_q8; with
 * NXG_GEMM_ACT63 for act_max 63, with NXG_GEMM_F32_IN for nxg_linear_f32_relu2_q8_rows, whose
 * shapes without the fused row-tile kernel, or with too few row tiles per workgroup, run the
 * quantize kernel, then the one named),
 * NXG_GEMM_SUMS (nxg_linear_i8_block_sums). A static string, or NULL for a shape or flag
 * combination the entry points refuse. */
#define NXG_GEMM_RESIDUAL 1
#define NXG_GEMM_RELU2    2
#define NXG_GEMM_SUMS     4
#define NXG_GEMM_ACT63    8
#define NXG_GEMM_F32_IN   16
NXG_API const char * nxg_gemm_kernel_name(int32_t T, int32_t n_in, int32_t n_out, int32_t flags, int32_t cus);

#ifdef __cplusplus
}
#endif

#endif /* NXG_LINEAR_H */
