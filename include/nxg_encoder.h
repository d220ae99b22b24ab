/* nxg_encoder.h -- the NexteraBERT encoder's forward pass on one GPU.
 *
 * A model context over libnxg's kernels: nxg_encoder_load reads a NexteraBERT GGUF file the
 * way nextera_load does (src/nexterabert.cpp:1549-1712: the same metadata keys and
 * defaults, the same int8 placement rule and weight expansion, conv kernels re-laid out
 * one row per tap), keeps every tensor the encoder reads resident on the device, and
 * nxg_encoder_encode runs builder::encoder (src/nexterabert.cpp:1270-1292) there: the
 * embedding lookup, per block its mixer (SnowLily, sliding-window or full attention, HRA)
 * and MLP, then out_norm; every linear on the int8 path. It stands where the reference's
 * run_forward (:1861-1935) builds and computes its ggml graph for nextera_encode /
 * nextera_encode_segments; each sequence's result does not depend on the rest of the
 * batch.
 *
 * Return codes are the reference C API's (nexterabert.h:38-123): 0 ok, 1 bad input, 2
 * allocation, 3 device (NXG_OK, NXG_EINVAL, NXG_ENOMEM, NXG_EDEVICE); nxg_last_error()
 * gives the reason the reference prints on stderr. A context is used by one host thread at
 * a time, as nextera_context.
 *
 * Not covered: the heads (pooler, classifier, MLM: nextera_pooler_output, nextera_classify,
 * nextera_mlm_logits), and files whose encoder linears are not all on the int8 path
 * (use_int8 = 0 or a weight the placement rule leaves to ggml): loading such a file fails
 * with NXG_EINVAL. Attention layers need head_dim 64.
 */
#ifndef NXG_ENCODER_H
#define NXG_ENCODER_H

#include <stddef.h>
#include <stdint.h>

#include "nxg_linear.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nxg_encoder nxg_encoder;

/* Load-time options (the GPU counterparts of struct nextera_params, nexterabert.h:29-34). */
typedef struct nxg_encoder_params {
    int32_t act_max;        /* 127: the VNNI build's activations (ACT_MAX, src/nexterabert.cpp:53-70); 63: the AVX2-only build's */
    int32_t load_threads;   /* host threads expanding weights; <= 0: all hardware threads (:1683) */
    int32_t verbosity;      /* 0 silent, 1 load summary on stderr */
} nxg_encoder_params;

NXG_API nxg_encoder_params nxg_encoder_default_params(void);

/* nextera_load (src/nexterabert.cpp:1549-1760) for the encoder. *out is NULL on failure. */
NXG_API int32_t nxg_encoder_load(const char * path, const nxg_encoder_params * params, nxg_encoder ** out);

/* nextera_free. */
NXG_API void nxg_encoder_free(nxg_encoder * e);

/* nextera_n_embd, nextera_n_vocab, nextera_n_layer, nextera_n_token_types (nexterabert.h:45-52). */
NXG_API int32_t nxg_encoder_n_embd(const nxg_encoder * e);
NXG_API int32_t nxg_encoder_n_vocab(const nxg_encoder * e);
NXG_API int32_t nxg_encoder_n_layer(const nxg_encoder * e);
NXG_API int32_t nxg_encoder_n_token_types(const nxg_encoder * e);

/* Device memory the context holds: weights, tables and the current work buffers. Not
 * counted: the NXG_NOALLOC_SCRATCH_BYTES array (nxg_linear.h) that loading the library
 * reserves on each GPU the process uses. */
NXG_API size_t nxg_encoder_device_bytes(const nxg_encoder * e);

/* Caps the work buffers at `bytes` (0: no cap; the default). The work area holds the
 * activations of the largest batch seen and the attention's score workspace; where the
 * whole does not fit under the cap or in the device's free memory, the workspace is halved
 * until it does, down to none (long documents then recompute their scores: same results,
 * slower). A batch whose activations alone exceed the cap fails with NXG_ENOMEM. No
 * counterpart in the reference, whose ggml allocator sizes its graph per call. */
NXG_API int32_t nxg_encoder_set_work_limit(nxg_encoder * e, int64_t bytes);

/* Bytes of attention score workspace in the current work area (0: none, or no pass yet). */
NXG_API int64_t nxg_encoder_attention_workspace(const nxg_encoder * e);

/* nextera_debug_set_layers (src/nexterabert.cpp:1815-1820): run only the first n_layers
 * blocks and return the residual stream before out_norm (-1: the full model). */
NXG_API void nxg_encoder_set_layers(nxg_encoder * e, int32_t n_layers);

/* nextera_encode_segments (nexterabert.h:80-99; nextera_encode with token_types NULL) on host
 * buffers:
 *   tokens       sum(lengths) ids, sequences concatenated
 *   token_types  NULL, or sum(lengths) segment ids (ignored when the file has no segment
 *                embeddings, as in the reference)
 *   lengths      n_seqs lengths, each >= 1
 *   hidden       out, optional: sum(lengths) * n_embd (last_hidden_state)
 *   pooled       out, optional: n_seqs * n_embd, the mean of each sequence's rows, or with
 *                normalize the L2-normalised sum */
NXG_API int32_t nxg_encoder_encode(nxg_encoder * e, const int32_t * tokens, const int32_t * token_types,
                                   const int32_t * lengths, int32_t n_seqs, float * hidden, float * pooled,
                                   int32_t normalize);

/* The same forward on device buffers, launched on `stream` (a hipStream_t; NULL: the
 * default stream) without synchronising: tokens / token_types device int32, hidden / pooled
 * device float (either may be NULL); lengths stay on the host. Token ids are not checked
 * here (the kernels clamp them into the table): the caller validates them. A call whose
 * lengths differ from the previous call's waits for `stream` and uploads the new offsets,
 * scales and RoPE tables (and may grow the work area); a call with the same lengths does
 * neither, so only such calls may be captured into a HIP graph. */
NXG_API int32_t nxg_encoder_forward(nxg_encoder * e, const int32_t * tokens, const int32_t * token_types,
                                    const int32_t * lengths, int32_t n_seqs, float * hidden, float * pooled,
                                    int32_t normalize, void * stream);

/* nextera_last_ms (nexterabert.h:121-122): wall time of the last nxg_encoder_encode, in ms. */
NXG_API double nxg_encoder_last_ms(const nxg_encoder * e);

/* The number of int8 linears the file's encoder has (before projections sharing an input are
 * fused): the count nextera_load reports in its system info (src/nexterabert.cpp:1735-1752). */
NXG_API int32_t nxg_encoder_n_int8(const nxg_encoder * e);

/* Kinds of launch the profiler tells apart, the reference's prof_kind (src/nexterabert.cpp:
 * 262-266): int8 linears (every GEMM, the MLP's fused c_fc -> relu^2 -> int8 included),
 * attention, the row ops (norms, convolutions, gates, DyT/RoPE, block means, quantizations,
 * pooling); OTHER is what the reference leaves to ggml (embedding rows, out_norm, copies). */
#define NXG_PROF_LINEAR 0
#define NXG_PROF_ATTN   1
#define NXG_PROF_ROWS   2
#define NXG_PROF_OTHER  3
#define NXG_PROF_COUNT  4

/* nextera_debug_profile (src/nexterabert.cpp:1823-1826): clears the profile and turns it on or
 * off. While it is on, every forward pass records a HIP event after each launch on its stream
 * and adds the device time of each launch to its kind; nxg_encoder_forward then waits for its
 * pass to end (so a profiled pass cannot be captured into a graph: NXG_EINVAL). */
NXG_API void nxg_encoder_profile(nxg_encoder * e, int32_t enable);

/* The profile so far: kind_ms [NXG_PROF_COUNT] device ms per kind, summed over the passes;
 * device_ms their total; wall_ms the host wall time of the nxg_encoder_encode calls (the
 * device time for nxg_encoder_forward passes); passes the number of profiled passes. Any
 * output may be NULL. */
NXG_API int32_t nxg_encoder_profile_read(const nxg_encoder * e, double * kind_ms, double * device_ms,
                                         double * wall_ms, int64_t * passes);

#ifdef __cplusplus
}
#endif

#endif /* NXG_ENCODER_H */
