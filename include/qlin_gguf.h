/*
 * qlin_gguf.h -- GGUF container reader and device weight residency (host side of libqlin).
 *
 * The reference engine opens a model file with GgufFile (AI/codes/local-llm/src/format/gguf/
 * GgufFile.cpp:152-247): it maps the file, parses the header, the metadata key/values and the tensor
 * table, reverses each tensor's dims to [outermost .. innermost] (a weight becomes [out_dim, in_dim])
 * and locates its packed bytes past the data section start, aligned to general.alignment (default 32).
 * CudaWeightPool::cached_weight (src/backend/cuda/mem/CudaWeightPool.cpp:119-175) then copies each
 * tensor to the device once, and expert slices of a packed [E, rows, cols] tensor are views into that
 * one copy (StorageTensor::slice, src/tensor/StorageTensor.cpp:23-44; RoutedExperts.cpp:23-32).
 * These entry points do the same, so that real .gguf files drive the kernels of qlin.h.
 *
 * Unlike the kernel entry points, the pool allocates device memory (hipMalloc) and copies
 * synchronously: it is model-load work, as the reference's weight pool is, never on the decode path.
 * Errors are qlin_status codes (qlin.h); the reference throws std::runtime_error in the same cases.
 */
#ifndef QLIN_GGUF_H
#define QLIN_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "qlin.h"

#ifdef __cplusplus
extern "C" {
#endif

#define QLIN_GGUF_MAX_DIMS 4

/* GGUF metadata value types (gguf_metadata_value_type), as GgufFile.h:47-61 lists them. */
enum qlin_gguf_value_type {
    QLIN_GGUF_U8 = 0, QLIN_GGUF_I8 = 1, QLIN_GGUF_U16 = 2, QLIN_GGUF_I16 = 3, QLIN_GGUF_U32 = 4,
    QLIN_GGUF_I32 = 5, QLIN_GGUF_F32 = 6, QLIN_GGUF_BOOL = 7, QLIN_GGUF_STRING = 8, QLIN_GGUF_ARRAY = 9,
    QLIN_GGUF_U64 = 10, QLIN_GGUF_I64 = 11, QLIN_GGUF_F64 = 12
};

typedef struct qlin_gguf qlin_gguf;

/* One entry of the tensor table.  Pointers stay valid until qlin_gguf_close. */
typedef struct qlin_gguf_tensor {
    const char *name;                    /* NUL-terminated */
    int type;                            /* ggml type code as stored */
    int n_dims;
    int64_t shape[QLIN_GGUF_MAX_DIMS];   /* the file's dims reversed: shape[0] outermost; unused = 1 */
    uint64_t nbytes;                     /* packed bytes */
    uint64_t offset;                     /* from the start of the data section */
    const uint8_t *data;                 /* host pointer into the mapped file */
} qlin_gguf_tensor;

/* Maps and parses a GGUF v2/v3 file (GgufFile.cpp:152-231).  QLIN_ERR_IO: cannot open or map;
 * QLIN_ERR_FORMAT: bad magic or version, a read past the end, an unknown tensor or value type, an
 * element count that is not a whole number of blocks, tensor data past the end of the file. */
int qlin_gguf_open(const char *path, qlin_gguf **out);
void qlin_gguf_close(qlin_gguf *g);
uint32_t qlin_gguf_version(const qlin_gguf *g);
uint32_t qlin_gguf_alignment(const qlin_gguf *g);

int64_t qlin_gguf_tensor_count(const qlin_gguf *g);
/* Index of the tensor called name, or -1 (GgufFile::contain_tensor_view / get_tensor_view). */
int64_t qlin_gguf_find_tensor(const qlin_gguf *g, const char *name);
int qlin_gguf_tensor_info(const qlin_gguf *g, int64_t index, qlin_gguf_tensor *out);

/* Metadata (GgufFile::metadata_value).  Keys are listed in file order.  Integers of every width and
 * bools read as int64, f32/f64 as double; a key of another type gives QLIN_ERR_NOT_FOUND. */
int64_t qlin_gguf_metadata_count(const qlin_gguf *g);
const char *qlin_gguf_metadata_key(const qlin_gguf *g, int64_t index);
int qlin_gguf_metadata_type(const qlin_gguf *g, const char *key); /* value type, or -1 if absent */
int qlin_gguf_get_i64(const qlin_gguf *g, const char *key, int64_t *out);
int qlin_gguf_get_f64(const qlin_gguf *g, const char *key, double *out);
int qlin_gguf_get_str(const qlin_gguf *g, const char *key, const char **out, size_t *len);
/* Arrays: element type and count, then elements by index (bool arrays read as int64). */
int qlin_gguf_get_array_info(const qlin_gguf *g, const char *key, int *elem_type, int64_t *count);
int qlin_gguf_get_array_i64(const qlin_gguf *g, const char *key, int64_t index, int64_t *out);
int qlin_gguf_get_array_f64(const qlin_gguf *g, const char *key, int64_t index, double *out);
int qlin_gguf_get_array_str(const qlin_gguf *g, const char *key, int64_t index, const char **out, size_t *len);

/* Device residency (CudaWeightPool).  A pool keeps one device copy per tensor name; destroying it
 * frees them all.  qlin_pool_weight uploads a tensor on first use and returns the cached copy after.
 * qlin_pool_expert_view returns expert e of a packed 3-D tensor [E, rows, cols]: the pool's copy of
 * the whole tensor plus e * (nbytes / E), with that expert's rows and cols (RoutedExperts.cpp:23-32).
 * QLIN_ERR_ALLOC: the device allocation or copy failed. */
typedef struct qlin_pool qlin_pool;
int qlin_pool_create(qlin_pool **out);
void qlin_pool_destroy(qlin_pool *p);
int qlin_pool_weight(qlin_pool *p, const qlin_gguf *g, const char *name, void **dev, uint64_t *nbytes);
int qlin_pool_expert_view(qlin_pool *p, const qlin_gguf *g, const char *name, int expert, void **dev,
                          uint64_t *expert_bytes, int64_t *rows, int64_t *cols);
uint64_t qlin_pool_resident_bytes(const qlin_pool *p);

#ifdef __cplusplus
}
#endif
#endif /* QLIN_GGUF_H */
