/* nxg_gguf.h -- GGUF model files for the int8 linear path.
 *
 * A reader of GGUF files (versions 2 and 3 of the published format: header, typed
 * key/value metadata, tensor table, aligned tensor data), written for this engine. It
 * stands where the reference calls ggml's gguf API while loading (nextera_load,
 * src/nexterabert.cpp:1549-1712: gguf_init_from_file, gguf_find_key/gguf_get_val_*,
 * gguf_get_tensor_name/offset, gguf_get_data_offset, then fread of each tensor). The file
 * is mapped read-only; tensor data pointers stay valid until nxg_gguf_close.
 *
 * Metadata value types and tensor types are GGUF's own numbering (tensor types: enum
 * nxg_type in nxg_linear.h). Tensor dimensions are ggml's ne[]: ne[0] is the row length.
 * Errors: NXG_EINVAL (malformed or unsupported file, bad index or type) or NXG_ENOMEM,
 * with the reason in nxg_last_error().
 */
#ifndef NXG_GGUF_H
#define NXG_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "nxg_linear.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF metadata value types. */
enum nxg_gguf_type {
    NXG_GGUF_UINT8 = 0, NXG_GGUF_INT8 = 1, NXG_GGUF_UINT16 = 2, NXG_GGUF_INT16 = 3,
    NXG_GGUF_UINT32 = 4, NXG_GGUF_INT32 = 5, NXG_GGUF_FLOAT32 = 6, NXG_GGUF_BOOL = 7,
    NXG_GGUF_STRING = 8, NXG_GGUF_ARRAY = 9, NXG_GGUF_UINT64 = 10, NXG_GGUF_INT64 = 11,
    NXG_GGUF_FLOAT64 = 12
};

typedef struct nxg_gguf nxg_gguf;

/* gguf_init_from_file (src/nexterabert.cpp:1557): parses the header, metadata and tensor
 * table and maps the file. Every tensor's data must lie inside the file. */
NXG_API int32_t nxg_gguf_open(const char * path, nxg_gguf ** out);
NXG_API void    nxg_gguf_close(nxg_gguf * g);

NXG_API uint32_t nxg_gguf_version(const nxg_gguf * g);
/* Start of the tensor data section (gguf_get_data_offset) and the alignment in force. */
NXG_API uint64_t nxg_gguf_data_offset(const nxg_gguf * g);
NXG_API uint32_t nxg_gguf_alignment(const nxg_gguf * g);

/* Metadata (gguf_find_key, gguf_get_val_*, gguf_get_arr_*). nxg_gguf_find_key returns the
 * key's index or -1. Scalar getters convert from any integer, float or bool type and fail
 * on strings and arrays; strings are returned with their length (not NUL-terminated in
 * the file; the pointer is to a NUL-terminated copy owned by g). */
NXG_API int64_t nxg_gguf_n_kv(const nxg_gguf * g);
NXG_API int64_t nxg_gguf_find_key(const nxg_gguf * g, const char * key);
NXG_API const char * nxg_gguf_key(const nxg_gguf * g, int64_t i);
NXG_API int32_t nxg_gguf_kv_type(const nxg_gguf * g, int64_t i);
NXG_API int32_t nxg_gguf_get_i64(const nxg_gguf * g, int64_t i, int64_t * v);
NXG_API int32_t nxg_gguf_get_f64(const nxg_gguf * g, int64_t i, double * v);
NXG_API int32_t nxg_gguf_get_str(const nxg_gguf * g, int64_t i, const char ** s, uint64_t * len);
/* Arrays: element type and count; elements by index (numbers as i64/f64, or strings). */
NXG_API int32_t nxg_gguf_arr_info(const nxg_gguf * g, int64_t i, int32_t * elem_type, uint64_t * n);
NXG_API int32_t nxg_gguf_arr_i64(const nxg_gguf * g, int64_t i, uint64_t j, int64_t * v);
NXG_API int32_t nxg_gguf_arr_f64(const nxg_gguf * g, int64_t i, uint64_t j, double * v);
NXG_API int32_t nxg_gguf_arr_str(const nxg_gguf * g, int64_t i, uint64_t j, const char ** s, uint64_t * len);

/* Tensor table (gguf_get_n_tensors, gguf_get_tensor_name, gguf_get_tensor_offset; shape
 * and type from the metadata context). ne[4] is filled with ones past n_dims; nbytes is
 * ggml_nbytes of the tensor. nxg_gguf_find_tensor returns the index or -1. */
NXG_API int64_t nxg_gguf_n_tensors(const nxg_gguf * g);
NXG_API int64_t nxg_gguf_find_tensor(const nxg_gguf * g, const char * name);
NXG_API const char * nxg_gguf_tensor_name(const nxg_gguf * g, int64_t i);
NXG_API int32_t nxg_gguf_tensor_info(const nxg_gguf * g, int64_t i, int32_t * type, int32_t * n_dims,
                                     int64_t * ne, uint64_t * offset, uint64_t * nbytes);
NXG_API const void * nxg_gguf_tensor_data(const nxg_gguf * g, int64_t i);

/* The int8 load of one tensor (src/nexterabert.cpp:1658-1667 and :1693-1696): checks the
 * placement rule (nxg_weight_is_int8 with use_int8 = 1), expands the tensor as
 * build_i8_weight (nxg_expand_weight, n_threads <= 0: all hardware threads) and uploads it
 * (nxg_weight_create). NXG_EINVAL if the tensor is not an int8 linear weight. */
NXG_API int32_t nxg_gguf_weight_create(const nxg_gguf * g, int64_t i, int32_t n_threads, nxg_weight ** out);

#ifdef __cplusplus
}
#endif

#endif /* NXG_GGUF_H */
