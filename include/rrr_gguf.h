/*
 * rrr_gguf.h -- bounds-checked GGUF v2/v3 reader and raw-weight upload of
 * librrr_hip.so (host code; the reader makes no HIP call).
 *
 * Replaces the reference's loader, src/model/gguf.rs, whose reader the decode
 * path depends on for every weight byte it uploads (phi4.rs:741-773).  The
 * file layout follows the published GGUF specification (ggml, docs/gguf.md):
 *
 *   header      magic "GGUF" (u32 0x46554747 LE), version u32, n_tensors u64,
 *               n_kv u64                                       (gguf.rs:131-135)
 *   metadata    n_kv x { key: u64 len + bytes, value type u32, value }
 *                                                              (gguf.rs:141-146)
 *   tensors     n_tensors x { name, n_dims u32, dims u64[n_dims] (ne0 first),
 *               ggml type u32, offset u64 }                    (gguf.rs:150-158)
 *   data        starts at the header end rounded up to general.alignment
 *               (default 32); each tensor at data start + offset (gguf.rs:161-163)
 *
 * Differences from gguf.rs, each a fix of something that reads the wrong
 * bytes or crashes there:
 *   - UINT8 / INT8 values are 1 byte (gguf.rs:100-101 reads 4, which shifts
 *     every later key and tensor record);
 *   - an unknown value type is an error (gguf.rs:119 skips one byte and goes on);
 *   - every read is bounds-checked against the file (gguf.rs indexes the
 *     mapping directly and panics or reads past a record);
 *   - tensor sizes come from the full ggml type table, and a row length that is
 *     not a whole number of blocks, or a tensor that ends past the file, is an
 *     error (gguf.rs:177-194 truncates n_elements / block and panics on the
 *     other types);
 *   - general.alignment must be a power of two and each tensor offset a
 *     multiple of it; duplicate keys and tensor names are errors (gguf.rs:145
 *     keeps the last one silently); keys and tensor names must be UTF-8.
 *
 * All pointers returned into the file (names, keys, values, tensor data) stay
 * valid until rrr_gguf_close().  A handle may be read from several threads at
 * once; rrr_gguf_close() must not race other calls on the same handle.
 */
#ifndef RRR_GGUF_H
#define RRR_GGUF_H

#include <stdint.h>

#include "rrr_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes of the reader, beside rrr_status. */
#define RRR_ERR_FORMAT (-11)    /* malformed or unsupported file contents */
#define RRR_ERR_NOT_FOUND (-12) /* no such key or tensor */
#define RRR_ERR_IO (-13)        /* open / stat / mmap failed */

/* Metadata value types (the GGUF specification's gguf_metadata_value_type). */
typedef enum rrr_gguf_value_type {
    RRR_GGUF_UINT8 = 0,
    RRR_GGUF_INT8 = 1,
    RRR_GGUF_UINT16 = 2,
    RRR_GGUF_INT16 = 3,
    RRR_GGUF_UINT32 = 4,
    RRR_GGUF_INT32 = 5,
    RRR_GGUF_FLOAT32 = 6,
    RRR_GGUF_BOOL = 7,
    RRR_GGUF_STRING = 8,
    RRR_GGUF_ARRAY = 9,
    RRR_GGUF_UINT64 = 10,
    RRR_GGUF_INT64 = 11,
    RRR_GGUF_FLOAT64 = 12
} rrr_gguf_value_type;

typedef struct rrr_gguf rrr_gguf;

/* One metadata pair (MetaValue, gguf.rs:28-38).  Values are little-endian and
 * may be unaligned: copy them out (memcpy) rather than dereferencing. */
typedef struct rrr_gguf_kv {
    const char *key;    /* NUL-terminated */
    uint64_t key_len;
    uint32_t type;      /* rrr_gguf_value_type */
    uint32_t elem_type; /* arrays: the element type; otherwise equal to type */
    uint64_t count;     /* arrays: elements; strings: bytes; scalars: 1 */
    const void *data;   /* scalar: the value; string: its bytes (not
                           NUL-terminated); array: the first element record */
    uint64_t bytes;     /* bytes at data (for arrays, all element records) */
} rrr_gguf_kv;

/* One tensor record (TensorInfo, gguf.rs:10-16) with its byte range resolved
 * (tensor_bytes, gguf.rs:173-195). */
typedef struct rrr_gguf_tensor {
    const char *name;   /* NUL-terminated */
    uint64_t name_len;
    uint32_t n_dims;    /* 1..4 */
    uint32_t type;      /* ggml type */
    uint64_t dims[4];   /* ne0 (innermost, the row length) first; unused = 1 */
    uint64_t offset;    /* from the start of the data section */
    uint64_t n_elements;
    uint64_t bytes;     /* storage bytes: n_elements / block_elems * block_bytes */
    const void *data;   /* the tensor's bytes inside the file mapping */
} rrr_gguf_tensor;

/* Maps and parses a GGUF file (GGUFModel::load, gguf.rs:125-170).  On success
 * *out owns the read-only mapping; close it with rrr_gguf_close(). */
int rrr_gguf_open(const char *path, rrr_gguf **out);

/* Parses a GGUF image already in memory.  The memory is borrowed: it must
 * stay valid and unchanged until rrr_gguf_close(). */
int rrr_gguf_open_memory(const void *data, uint64_t bytes, rrr_gguf **out);

/* Unmaps and frees; NULL is accepted.  RRR_ERR_STALE for a closed handle. */
int rrr_gguf_close(rrr_gguf *g);

/* GGUFModel's version, n_tensors, metadata.len(), data_offset (gguf.rs:18-25)
 * and the alignment in effect.  Any output pointer may be NULL. */
int rrr_gguf_header(const rrr_gguf *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv,
                    uint64_t *alignment, uint64_t *data_offset);

/* Metadata pair `index` in file order, or the index of `key`
 * (metadata.get(key), gguf.rs:21; RRR_ERR_NOT_FOUND if absent). */
int rrr_gguf_kv_at(const rrr_gguf *g, uint64_t index, rrr_gguf_kv *out);
int rrr_gguf_find_kv(const rrr_gguf *g, const char *key, uint64_t *index);

/* Strings first .. first + count - 1 of a string array (or, with first = 0
 * and count = 1, a string scalar): pointers into the file and byte lengths.
 * Used for tokenizer.ggml.tokens / merges (tokenizer.rs:18-40). */
int rrr_gguf_kv_strings(const rrr_gguf *g, uint64_t index, uint64_t first, uint64_t count,
                        const char **ptrs, uint64_t *lens);

/* Typed reads of a scalar value (MetaValue::as_u64 / as_f32 / as_str,
 * gguf.rs:41-59).  get_u64 takes any integer type (a negative signed value is
 * RRR_ERR_INVALID_ARG, where as_u64 wraps it); get_f64 takes FLOAT32 and
 * FLOAT64; get_str takes STRING.  A key of another type is RRR_ERR_BAD_TYPE
 * (as_* returns None there), a missing key RRR_ERR_NOT_FOUND. */
int rrr_gguf_get_u64(const rrr_gguf *g, const char *key, uint64_t *value);
int rrr_gguf_get_f64(const rrr_gguf *g, const char *key, double *value);
int rrr_gguf_get_str(const rrr_gguf *g, const char *key, const char **str, uint64_t *len);

/* Tensor record `index` in file order, or by name (tensor_infos lookup +
 * tensor_bytes, gguf.rs:173-195; RRR_ERR_NOT_FOUND if absent). */
int rrr_gguf_tensor_at(const rrr_gguf *g, uint64_t index, rrr_gguf_tensor *out);
int rrr_gguf_find_tensor(const rrr_gguf *g, const char *name, rrr_gguf_tensor *out);

/* Block geometry of a ggml type (the size table behind tensor_bytes,
 * gguf.rs:178-191, completed to every type ggml defines): elements per block
 * and bytes per block.  RRR_ERR_BAD_TYPE for an unknown or retired type. */
int rrr_gguf_type_size(uint32_t ggml_type, uint32_t *block_elems, uint32_t *block_bytes);

/* Uploads tensor `name` to the device unchanged as a weight of K = ne0 and
 * N = ne1 * ne2 * ne3 rows (rrr_weight_upload): the raw-byte path that
 * replaces load_weight_gpu's tensor_bytes + repack + upload (phi4.rs:741-773).
 * The type must be one the kernels read (F32, Q4_K, Q5_K, Q6_K; else
 * RRR_ERR_BAD_TYPE naming the tensor) and ne0 a multiple of 256. */
int rrr_gguf_upload(rrr_ctx *ctx, const rrr_gguf *g, const char *name, rrr_buf **out);

#ifdef __cplusplus
}
#endif
#endif
