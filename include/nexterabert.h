/* nexterabert.h -- the public C API of NexteraBERT.cpp (src/nexterabert.h:28-123 of the
 * reference), served by the MI355X (gfx950) engine: libnexterabert.so in this build, a thin
 * layer over the GPU encoder of nxg_encoder.h. A program written against the reference's
 * header compiles against this one unchanged and links against libnexterabert.so; the
 * declarations, the struct layout, the return codes (0 ok, 1 bad input, 2 allocation,
 * 3 compute) and the NULL-on-failure load are the reference's.
 *
 * What differs, and why:
 *   - nextera_params.use_int8 = 0 asks for ggml's float/quantized kernels, which this engine
 *     does not have: nextera_load refuses it (NULL, reason on stderr). use_repack only
 *     concerns ggml's repacking and is ignored.
 *   - n_threads (nextera_load, nextera_set_n_threads) sets the host threads that expand the
 *     weights at load; the forward pass runs on the GPU. <= 0 means the reference's default,
 *     all logical cores but about 10% (src/nexterabert.cpp:1519-1524).
 *   - The heads (nextera_pooler_output, nextera_classify, nextera_mlm_logits) are not built:
 *     with the head present in the file they return 1 with the reason on stderr; without
 *     it, 1 with the reference's own message.
 *   - The int8 path computes with the reference's VNNI numerics (ACT_MAX 127); results are
 *     bit-identical to this build's restatement of that path (oracle/ in the repository).
 * A context is used by one host thread at a time, as the reference's.
 */
#ifndef NEXTERABERT_H
#define NEXTERABERT_H

#include <stddef.h>
#include <stdint.h>

/* NEXTERA_API as the reference defines it: exported from the shared library when
 * NEXTERA_SHARED is set (NEXTERA_BUILD while building it). */
#if defined(NEXTERA_SHARED)
#  if defined(_WIN32)
#    if defined(NEXTERA_BUILD)
#      define NEXTERA_API __declspec(dllexport)
#    else
#      define NEXTERA_API __declspec(dllimport)
#    endif
#  else
#    define NEXTERA_API __attribute__((visibility("default")))
#  endif
#else
#  define NEXTERA_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

struct nextera_context;

struct nextera_params {
    int32_t n_threads;   /* host threads for the load-time weight expansion; <= 0: hw - hw/10 */
    int32_t use_int8;    /* must be 1: every encoder linear runs on the GPU int8 GEMM */
    int32_t use_repack;  /* ggml's repacking; ignored */
    int32_t verbosity;   /* 0 silent, 1 load summary on stderr */
};

/* n_threads 0, use_int8 1, use_repack 1, verbosity 0. */
NEXTERA_API struct nextera_params nextera_default_params(void);

/* Reads a NexteraBERT GGUF file and puts its encoder on the current HIP device. NULL on
 * failure, with the reason on stderr. */
NEXTERA_API struct nextera_context * nextera_load(const char * path, struct nextera_params params);
NEXTERA_API void nextera_free(struct nextera_context * ctx);

/* Metadata of the loaded file (nextera_load's hparams). */
NEXTERA_API int32_t nextera_n_embd(const struct nextera_context * ctx);
NEXTERA_API int32_t nextera_n_vocab(const struct nextera_context * ctx);
NEXTERA_API int32_t nextera_n_layer(const struct nextera_context * ctx);
NEXTERA_API int32_t nextera_has_mlm_head(const struct nextera_context * ctx);
/* Heads the file carries: the pooler, and a classifier whose task is "" or one of
 * "sequence-classification", "multiple-choice", "token-classification", "question-answering". */
NEXTERA_API int32_t nextera_has_pooler(const struct nextera_context * ctx);
NEXTERA_API int32_t nextera_n_token_types(const struct nextera_context * ctx);   /* 0: no segment embeddings */
NEXTERA_API const char * nextera_classifier_task(const struct nextera_context * ctx);
NEXTERA_API int32_t nextera_n_labels(const struct nextera_context * ctx);
/* Label i's name from the file ("" when it has none). */
NEXTERA_API const char * nextera_label(const struct nextera_context * ctx, int32_t i);
NEXTERA_API int32_t nextera_token_cls(const struct nextera_context * ctx);
NEXTERA_API int32_t nextera_token_sep(const struct nextera_context * ctx);
NEXTERA_API int32_t nextera_token_pad(const struct nextera_context * ctx);
NEXTERA_API int32_t nextera_token_mask(const struct nextera_context * ctx);
/* The tokenizer.json stored in the file ("" when absent). */
NEXTERA_API const char * nextera_tokenizer_json(const struct nextera_context * ctx);
/* The file type named from general.file_type, e.g. "Q4_K_M". */
NEXTERA_API const char * nextera_ftype(const struct nextera_context * ctx);
/* The device and the engine's int8 path, one line. */
NEXTERA_API const char * nextera_system_info(const struct nextera_context * ctx);

NEXTERA_API void    nextera_set_n_threads(struct nextera_context * ctx, int32_t n_threads);
NEXTERA_API int32_t nextera_get_n_threads(const struct nextera_context * ctx);

/* One forward pass over n_seqs token sequences, unpadded:
 *   tokens     sum(lengths) ids, the sequences one after another (special tokens included)
 *   lengths    n_seqs lengths, each >= 1
 *   hidden     out, optional: sum(lengths) * n_embd floats, last_hidden_state
 *   pooled     out, optional: n_seqs * n_embd floats, each sequence's mean row
 *   normalize  1: pooled vectors L2-normalised
 * A sequence's outputs are the same bits whatever else is in the batch. Returns 0 on success. */
NEXTERA_API int32_t nextera_encode(struct nextera_context * ctx,
                                   const int32_t * tokens, const int32_t * lengths, int32_t n_seqs,
                                   float * hidden, float * pooled, int32_t normalize);

/* nextera_encode with token_types: NULL, or sum(lengths) segment ids, added through the
 * file's segment embeddings (ignored when the file has none). */
NEXTERA_API int32_t nextera_encode_segments(struct nextera_context * ctx,
                                            const int32_t * tokens, const int32_t * token_types,
                                            const int32_t * lengths, int32_t n_seqs,
                                            float * hidden, float * pooled, int32_t normalize);

/* The heads (not built by this engine; see above). out / logits: as the reference's. */
NEXTERA_API int32_t nextera_pooler_output(struct nextera_context * ctx,
                                          const int32_t * tokens, const int32_t * token_types,
                                          const int32_t * lengths, int32_t n_seqs, float * out);
NEXTERA_API int32_t nextera_classify(struct nextera_context * ctx,
                                     const int32_t * tokens, const int32_t * token_types,
                                     const int32_t * lengths, int32_t n_seqs, float * logits);
NEXTERA_API int32_t nextera_mlm_logits(struct nextera_context * ctx,
                                       const int32_t * tokens, int32_t n_tokens,
                                       const int32_t * positions, int32_t n_pos,
                                       float * logits);

/* Wall time of the last nextera_encode / nextera_encode_segments call, in ms. */
NEXTERA_API double nextera_last_ms(const struct nextera_context * ctx);

/* Diagnostics the reference exports outside its public header (src/nexterabert.cpp:1815-1841;
 * python/nexterabert_cpp.py:83 and tools/cli.cpp:22-26 declare them themselves):
 *   nextera_debug_set_layers     run only the first n_layers blocks and return the residual
 *                                stream before out_norm (-1: the whole model)
 *   nextera_debug_profile        clear the profile and turn it on (1) or off (0)
 *   nextera_debug_profile_print  per-pass ms of the int8 linears, attention and row ops (GPU
 *                                time from HIP events), the rest of the wall time, and the
 *                                total, on stderr */
NEXTERA_API void nextera_debug_set_layers(struct nextera_context * ctx, int32_t n_layers);
NEXTERA_API void nextera_debug_profile(struct nextera_context * ctx, int32_t enable);
NEXTERA_API void nextera_debug_profile_print(const struct nextera_context * ctx);

#ifdef __cplusplus
}
#endif

#endif /* NEXTERABERT_H */
