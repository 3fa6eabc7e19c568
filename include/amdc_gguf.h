/* amdc_gguf.h -- the on-disk side of the quantized GEMV path: a GGUF v3
 * reader and the load of its quantized matrices into the CDNA4 layout
 * (amdc_q4.h) on the device. Part of libamdc_q4.so.
 *
 * Replaces the reference's src/gguf.c (gguf_open / gguf_find /
 * gguf_get_int / gguf_get_float / gguf_get_str / gguf_tensor_find /
 * ggml_nbytes, src/gguf.h:56-68) and, for the matrix kinds of this path, the
 * load_mat_src + gpu_sink pair (src/model.c:401-494, src/hip.c:274-309) that
 * repacks a tensor and copies it to the device. Unlike the reference's reader,
 * which exits the process on a malformed file, every function here returns an
 * error code (amdc_last_error() says why): a library must not end its host.
 *
 * The file is memory-mapped; tensor data pointers point into the mapping and
 * stay valid until amdc_gguf_close. Little-endian hosts only (as the
 * reference). */
#ifndef AMDC_GGUF_H
#define AMDC_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF value types (the GGUF v3 specification; src/gguf.h:8-11). */
enum {
  AMDC_GGUF_U8 = 0, AMDC_GGUF_I8 = 1, AMDC_GGUF_U16 = 2, AMDC_GGUF_I16 = 3, AMDC_GGUF_U32 = 4, AMDC_GGUF_I32 = 5,
  AMDC_GGUF_F32 = 6, AMDC_GGUF_BOOL = 7, AMDC_GGUF_STR = 8, AMDC_GGUF_ARR = 9, AMDC_GGUF_U64 = 10, AMDC_GGUF_I64 = 11,
  AMDC_GGUF_F64 = 12
};

typedef struct amdc_gguf amdc_gguf;

typedef struct {
  const char *name;  /* 0-terminated, owned by the handle */
  uint32_t type;     /* GGML type id (0 F32, 1 F16, 2 Q4_0, 8 Q8_0, 12 Q4_K, 14 Q6_K, ...) */
  uint32_t n_dims;   /* 1..4 */
  uint64_t ne[4];    /* ne[0] is the contiguous dimension (the columns of a matrix); unused dims are 1 */
  uint64_t offset;   /* from the start of the data section */
  uint64_t nbytes;   /* 0 for a type the reader does not size */
  const void *data;  /* into the mapping; NULL when nbytes is 0 */
} amdc_gguf_tensor;

/* Open and parse (bounds-checked against the file size): header, key/value
 * pairs, tensor table; general.alignment (U32, a power of two, default 32)
 * places the data section. Tensors of known types must be aligned and inside
 * the file. Replaces gguf_open (src/gguf.c:131-194). */
int amdc_gguf_open(const char *path, amdc_gguf **out);
void amdc_gguf_close(amdc_gguf *g);

uint32_t amdc_gguf_version(const amdc_gguf *g);
uint32_t amdc_gguf_alignment(const amdc_gguf *g);
uint64_t amdc_gguf_data_offset(const amdc_gguf *g);
uint64_t amdc_gguf_n_kv(const amdc_gguf *g);
uint64_t amdc_gguf_n_tensors(const amdc_gguf *g);

/* Key i and its value type. */
int amdc_gguf_key_at(const amdc_gguf *g, uint64_t i, const char **key, uint32_t *type);
/* Scalars (gguf_get_int / gguf_get_float, src/gguf.c:212-242): 1 if the key
 * exists with a numeric type (integers and bool; floats for get_float, which
 * also converts integers), else 0. */
int amdc_gguf_get_int(const amdc_gguf *g, const char *key, int64_t *out);
int amdc_gguf_get_float(const amdc_gguf *g, const char *key, double *out);
/* A string value: pointer into the file (not 0-terminated) and length; 1 if
 * found and a string (gguf_get_str, :244-247, without the copy). */
int amdc_gguf_get_str(const amdc_gguf *g, const char *key, const char **p, uint64_t *n);
/* An array value: element type, count and, for arrays of scalars, the first
 * element in the file (little endian, packed); NULL data for arrays of
 * strings (read them with amdc_gguf_get_arr_str) and of arrays. */
int amdc_gguf_get_arr(const amdc_gguf *g, const char *key, uint32_t *elem_type, uint64_t *n, const void **data);
int amdc_gguf_get_arr_str(const amdc_gguf *g, const char *key, uint64_t i, const char **p, uint64_t *n);

/* Tensor i, or the index of a tensor by name (-1 if absent; gguf_tensor_find,
 * :249-253). */
int amdc_gguf_tensor_at(const amdc_gguf *g, uint64_t i, amdc_gguf_tensor *out);
int64_t amdc_gguf_find_tensor(const amdc_gguf *g, const char *name);

/* Bytes of n elements of a GGML type, 0 if unknown or n is not a whole number
 * of blocks (ggml_nbytes, :103-117). */
uint64_t amdc_ggml_nbytes(uint32_t type, uint64_t n);

/* ---------------------------------------------------------------- matrices */

/* A matrix of the quantized path in the CDNA4 layout. */
typedef struct {
  int kind;          /* AMDC_KIND_* (amdc_q4.h) */
  uint32_t rows, cols, nb;
  uint64_t bytes;    /* amdc_mat_bytes(kind, rows, cols) */
  void *w;           /* device memory (amdc_gguf_load), or NULL */
} amdc_mat;

/* The matrix kind of a GGML type for this path (Q4_0, Q8_0, Q4_K, Q6_K; the
 * reference's load_mat_src choice for a non-embedding matrix, src/model.c:
 * 406-470), -1 for the others (F32, F16, Q5_K, IQ*: not on this path). */
int amdc_gguf_mat_kind(uint32_t ggml_type);

/* Describe tensor `name` as a matrix (rows = ne[1], cols = ne[0]; ne[2] and
 * ne[3] must be 1) and check it against the kind's shape rules. */
int amdc_gguf_mat_info(const amdc_gguf *g, const char *name, amdc_mat *m);

/* Repack tensor `name` into host memory dst (m->bytes after amdc_gguf_mat_info)
 * with nthreads threads (0: one per MiB of weights, at most 16); the same
 * bytes as amdc_repack_q4 / _q8 / _q4k / _q6k of the whole matrix. Host only. */
int amdc_gguf_repack(const amdc_gguf *g, const char *name, int nthreads, amdc_mat *m, uint8_t *dst);

/* The streaming load (the reference's gpu_sink): allocate m->w on the device
 * and fill it with the repacked matrix in chunks of rows: nthreads threads
 * repack a chunk into one of two pinned staging buffers while the previous
 * chunk's copy runs on `stream` (NULL: the default stream); returns when the
 * matrix is on the device. The staging buffers (2 x 32 MiB by default,
 * AMDC_LOAD_CHUNK_KB) stay allocated for later loads until amdc_close; loads
 * must not run concurrently. Free the matrix with amdc_mat_release. */
int amdc_gguf_load(const amdc_gguf *g, const char *name, int nthreads, amdc_mat *m, void *stream);
int amdc_mat_release(amdc_mat *m);

#ifdef __cplusplus
}
#endif
#endif
