/* amdc_gguf.c -- the GGUF v3 reader of libamdc_q4.so and the host side of
 * the matrix load (include/amdc_gguf.h). The device side, the streaming copy,
 * is amdc_gguf_load in amdc_host.c.
 *
 * Format (GGUF v3, as the reference reads it, src/gguf.c:131-194): u32 magic
 * "GGUF", u32 version, u64 n_tensors, u64 n_kv; n_kv pairs (string key, u32
 * type, value: scalars little endian, strings as u64 length + bytes, arrays as
 * u32 element type + u64 count + elements); n_tensors entries (string name,
 * u32 n_dims, u64 ne[n_dims], u32 GGML type, u64 offset); then the data
 * section at the next multiple of general.alignment. Every read is checked
 * against the end of the file before it is made. */
#define _GNU_SOURCE
#include "../../include/amdc_gguf.h"

#include <fcntl.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/amdc_q4.h"
#include "amdc_internal.h"
#include "amdc_layout.h"

typedef uint32_t u32;
typedef uint64_t u64;

static int gfail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  amdc_fail_v(code, fmt, ap);
  va_end(ap);
  return code;
}

typedef struct {
  char *key;
  u32 type;
  u64 pos;      /* the value's first byte in the file */
  u64 u;        /* unsigned scalars and bool */
  int64_t i;    /* signed scalars */
  double f;     /* float scalars */
  u64 sp, sn;   /* a string: position and length */
  u32 at;       /* arrays: element type, count, first element */
  u64 an, apos;
  u64 *astr;    /* arrays of strings: the position of each string's length field */
} kv_t;

struct amdc_gguf {
  uint8_t *map;
  u64 size;
  u32 version, alignment;
  u64 n_kv, n_t, data_off;
  kv_t *kv;
  amdc_gguf_tensor *t;
};

typedef struct {
  const uint8_t *p;
  u64 pos, size;
  int err;
} rd;

static int need(rd *r, u64 n) {
  if (r->err || n > r->size || r->pos > r->size - n) {
    r->err = 1;
    return 0;
  }
  return 1;
}
static u64 get(rd *r, int n) {
  u64 v = 0;
  if (!need(r, (u64)n)) return 0;
  memcpy(&v, r->p + r->pos, (size_t)n);
  r->pos += (u64)n;
  return v;
}
/* a string: its length field and bytes; returns the position of the bytes */
static u64 get_str(rd *r, u64 *len) {
  *len = get(r, 8);
  if (!need(r, *len)) return 0;
  const u64 at = r->pos;
  r->pos += *len;
  return at;
}

static int scalar_bytes(u32 t) {
  switch (t) {
    case AMDC_GGUF_U8: case AMDC_GGUF_I8: case AMDC_GGUF_BOOL: return 1;
    case AMDC_GGUF_U16: case AMDC_GGUF_I16: return 2;
    case AMDC_GGUF_U32: case AMDC_GGUF_I32: case AMDC_GGUF_F32: return 4;
    case AMDC_GGUF_U64: case AMDC_GGUF_I64: case AMDC_GGUF_F64: return 8;
    default: return 0;
  }
}

/* skip (depth > 0) or read a value of type t */
static void value(rd *r, u32 t, kv_t *kv, int depth) {
  if (depth > 8) {
    r->err = 2;
    return;
  }
  if (t == AMDC_GGUF_STR) {
    u64 n;
    const u64 at = get_str(r, &n);
    if (kv) kv->sp = at, kv->sn = n;
    return;
  }
  if (t == AMDC_GGUF_ARR) {
    const u32 at = (u32)get(r, 4);
    const u64 n = get(r, 8);
    if (kv) kv->at = at, kv->an = n, kv->apos = r->pos;
    if (at == AMDC_GGUF_STR || at == AMDC_GGUF_ARR) {
      if (n > r->size / 8u) { /* every element takes at least 8 bytes */
        r->err = 1;
        return;
      }
      if (kv && at == AMDC_GGUF_STR) {
        kv->astr = malloc((n ? n : 1) * sizeof(u64));
        if (!kv->astr) {
          r->err = 3;
          return;
        }
      }
      for (u64 i = 0; i < n && !r->err; i++) {
        if (kv && kv->astr) kv->astr[i] = r->pos;
        value(r, at, NULL, depth + 1);
      }
      return;
    }
    const int sb = scalar_bytes(at);
    if (!sb || n > r->size / (u64)sb) {
      r->err = sb ? 1 : 2;
      return;
    }
    if (need(r, n * (u64)sb)) r->pos += n * (u64)sb;
    return;
  }
  const int sb = scalar_bytes(t);
  if (!sb) {
    r->err = 2;
    return;
  }
  const u64 raw = get(r, sb);
  if (!kv) return;
  switch (t) {
    case AMDC_GGUF_I8: kv->i = (int8_t)raw; break;
    case AMDC_GGUF_I16: kv->i = (int16_t)raw; break;
    case AMDC_GGUF_I32: kv->i = (int32_t)raw; break;
    case AMDC_GGUF_I64: kv->i = (int64_t)raw; break;
    case AMDC_GGUF_F32: {
      float f;
      const u32 b = (u32)raw;
      memcpy(&f, &b, 4);
      kv->f = f;
      break;
    }
    case AMDC_GGUF_F64: memcpy(&kv->f, &raw, 8); break;
    default: kv->u = raw;
  }
}

uint64_t amdc_ggml_nbytes(uint32_t type, uint64_t n) {
  /* bytes per block and weights per block of each GGML type */
  u64 bb, bw;
  switch (type) {
    case 0: bb = 4, bw = 1; break;     /* F32 */
    case 1: case 30: bb = 2, bw = 1; break; /* F16, BF16 */
    case 2: bb = 18, bw = 32; break;   /* Q4_0 */
    case 8: bb = 34, bw = 32; break;   /* Q8_0 */
    case 12: bb = 144, bw = 256; break; /* Q4_K */
    case 13: bb = 176, bw = 256; break; /* Q5_K */
    case 14: bb = 210, bw = 256; break; /* Q6_K */
    case 21: bb = 110, bw = 256; break; /* IQ3_S */
    case 23: bb = 136, bw = 256; break; /* IQ4_XS */
    default: return 0;
  }
  if (n % bw || n / bw > UINT64_MAX / bb) return 0;
  return n / bw * bb;
}

void amdc_gguf_close(amdc_gguf *g) {
  if (!g) return;
  for (u64 i = 0; g->kv && i < g->n_kv; i++) free(g->kv[i].key), free(g->kv[i].astr);
  for (u64 i = 0; g->t && i < g->n_t; i++) free((char *)g->t[i].name);
  free(g->kv);
  free(g->t);
  if (g->map && g->map != MAP_FAILED) munmap(g->map, g->size ? g->size : 1);
  free(g);
}

static char *dup_at(const uint8_t *p, u64 n) {
  char *c = malloc(n + 1);
  if (c) memcpy(c, p, n), c[n] = 0;
  return c;
}

int amdc_gguf_open(const char *path, amdc_gguf **out) {
  if (!path || !out) return gfail(AMDC_EINVAL, "gguf_open: null argument");
  *out = NULL;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return gfail(AMDC_EINVAL, "gguf_open: cannot open %s", path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return gfail(AMDC_EINVAL, "gguf_open: cannot stat %s", path);
  }
  amdc_gguf *g = calloc(1, sizeof *g);
  if (!g) {
    close(fd);
    return gfail(AMDC_EINVAL, "gguf_open: out of memory");
  }
  g->size = (u64)st.st_size;
  g->map = mmap(NULL, g->size ? g->size : 1, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (g->map == MAP_FAILED) {
    g->map = NULL;
    amdc_gguf_close(g);
    return gfail(AMDC_EINVAL, "gguf_open: cannot map %s", path);
  }
  rd r = {g->map, 0, g->size, 0};
  const u64 magic = get(&r, 4);
  g->version = (u32)get(&r, 4);
  g->n_t = get(&r, 8);
  g->n_kv = get(&r, 8);
  int rc = AMDC_OK;
  if (r.err) rc = gfail(AMDC_EINVAL, "%s: truncated GGUF header", path);
  else if (magic != 0x46554747u) rc = gfail(AMDC_EINVAL, "%s: not a GGUF file", path);
  else if (g->version != 3) rc = gfail(AMDC_EINVAL, "%s: GGUF version %u (only 3 is read)", path, g->version);
  else if (g->n_kv > g->size / 8u || g->n_t > g->size / 8u) rc = gfail(AMDC_EINVAL, "%s: bad key or tensor count", path);
  if (!rc) {
    g->kv = calloc(g->n_kv ? g->n_kv : 1, sizeof(kv_t));
    g->t = calloc(g->n_t ? g->n_t : 1, sizeof(amdc_gguf_tensor));
    if (!g->kv || !g->t) rc = gfail(AMDC_EINVAL, "gguf_open: out of memory");
  }
  g->alignment = 32;
  for (u64 i = 0; !rc && i < g->n_kv; i++) {
    kv_t *kv = &g->kv[i];
    u64 n;
    const u64 at = get_str(&r, &n);
    if (!r.err) kv->key = dup_at(g->map + at, n);
    kv->type = (u32)get(&r, 4);
    kv->pos = r.pos;
    if (!r.err) value(&r, kv->type, kv, 0);
    if (r.err == 3 || (!r.err && !kv->key)) rc = gfail(AMDC_EINVAL, "gguf_open: out of memory");
    else if (r.err == 2) rc = gfail(AMDC_EINVAL, "%s: key %llu: bad value type", path, (unsigned long long)i);
    else if (r.err) rc = gfail(AMDC_EINVAL, "%s: truncated GGUF (key %llu)", path, (unsigned long long)i);
    else if (strcmp(kv->key, "general.alignment") == 0 && kv->type == AMDC_GGUF_U32) g->alignment = (u32)kv->u;
  }
  if (!rc && (g->alignment == 0 || (g->alignment & (g->alignment - 1u))))
    rc = gfail(AMDC_EINVAL, "%s: general.alignment %u is not a power of two", path, g->alignment);
  for (u64 i = 0; !rc && i < g->n_t; i++) {
    amdc_gguf_tensor *t = &g->t[i];
    u64 n;
    const u64 at = get_str(&r, &n);
    if (!r.err) t->name = dup_at(g->map + at, n);
    t->n_dims = (u32)get(&r, 4);
    if (!r.err && (t->n_dims < 1u || t->n_dims > 4u)) {
      rc = gfail(AMDC_EINVAL, "%s: tensor %s has %u dimensions", path, t->name ? t->name : "?", t->n_dims);
      break;
    }
    u64 ne = 1;
    for (u32 d = 0; d < 4u; d++) t->ne[d] = 1;
    for (u32 d = 0; d < t->n_dims && !r.err; d++) {
      t->ne[d] = get(&r, 8);
      if (t->ne[d] && ne > UINT64_MAX / t->ne[d]) {
        rc = gfail(AMDC_EINVAL, "%s: tensor %s is too large", path, t->name ? t->name : "?");
        break;
      }
      ne *= t->ne[d];
    }
    t->type = (u32)get(&r, 4);
    t->offset = get(&r, 8);
    if (!rc && r.err) rc = gfail(AMDC_EINVAL, "%s: truncated GGUF (tensor %llu)", path, (unsigned long long)i);
    else if (!rc && !t->name) rc = gfail(AMDC_EINVAL, "gguf_open: out of memory");
    if (!rc) t->nbytes = amdc_ggml_nbytes(t->type, ne);
  }
  if (!rc) {
    g->data_off = (r.pos + g->alignment - 1u) / g->alignment * g->alignment;
    for (u64 i = 0; i < g->n_t; i++) {
      amdc_gguf_tensor *t = &g->t[i];
      if (!t->nbytes) continue; /* a type the reader does not size: refused when used */
      if (t->offset % g->alignment) {
        rc = gfail(AMDC_EINVAL, "%s: tensor %s is not aligned to %u", path, t->name, g->alignment);
        break;
      }
      if (g->data_off > g->size || t->offset > g->size - g->data_off || t->nbytes > g->size - g->data_off - t->offset) {
        rc = gfail(AMDC_EINVAL, "%s: tensor %s lies outside the file", path, t->name);
        break;
      }
      t->data = g->map + g->data_off + t->offset;
    }
  }
  if (rc) {
    amdc_gguf_close(g);
    return rc;
  }
  *out = g;
  return AMDC_OK;
}

uint32_t amdc_gguf_version(const amdc_gguf *g) { return g ? g->version : 0; }
uint32_t amdc_gguf_alignment(const amdc_gguf *g) { return g ? g->alignment : 0; }
uint64_t amdc_gguf_data_offset(const amdc_gguf *g) { return g ? g->data_off : 0; }
uint64_t amdc_gguf_n_kv(const amdc_gguf *g) { return g ? g->n_kv : 0; }
uint64_t amdc_gguf_n_tensors(const amdc_gguf *g) { return g ? g->n_t : 0; }

int amdc_gguf_key_at(const amdc_gguf *g, uint64_t i, const char **key, uint32_t *type) {
  if (!g || i >= g->n_kv) return gfail(AMDC_EINVAL, "gguf_key_at: no key %llu", (unsigned long long)i);
  if (key) *key = g->kv[i].key;
  if (type) *type = g->kv[i].type;
  return AMDC_OK;
}

static const kv_t *find(const amdc_gguf *g, const char *key) {
  for (u64 i = 0; g && key && i < g->n_kv; i++)
    if (strcmp(g->kv[i].key, key) == 0) return &g->kv[i];
  return NULL;
}

int amdc_gguf_get_int(const amdc_gguf *g, const char *key, int64_t *out) {
  const kv_t *kv = find(g, key);
  if (!kv) return 0;
  switch (kv->type) {
    case AMDC_GGUF_U8: case AMDC_GGUF_U16: case AMDC_GGUF_U32: case AMDC_GGUF_U64: case AMDC_GGUF_BOOL:
      if (out) *out = (int64_t)kv->u;
      return 1;
    case AMDC_GGUF_I8: case AMDC_GGUF_I16: case AMDC_GGUF_I32: case AMDC_GGUF_I64:
      if (out) *out = kv->i;
      return 1;
    default: return 0;
  }
}

int amdc_gguf_get_float(const amdc_gguf *g, const char *key, double *out) {
  const kv_t *kv = find(g, key);
  if (!kv) return 0;
  if (kv->type == AMDC_GGUF_F32 || kv->type == AMDC_GGUF_F64) {
    if (out) *out = kv->f;
    return 1;
  }
  int64_t v;
  if (!amdc_gguf_get_int(g, key, &v)) return 0;
  if (out) *out = (double)v;
  return 1;
}

int amdc_gguf_get_str(const amdc_gguf *g, const char *key, const char **p, uint64_t *n) {
  const kv_t *kv = find(g, key);
  if (!kv || kv->type != AMDC_GGUF_STR) return 0;
  if (p) *p = (const char *)g->map + kv->sp;
  if (n) *n = kv->sn;
  return 1;
}

int amdc_gguf_get_arr(const amdc_gguf *g, const char *key, uint32_t *elem_type, uint64_t *n, const void **data) {
  const kv_t *kv = find(g, key);
  if (!kv || kv->type != AMDC_GGUF_ARR) return 0;
  if (elem_type) *elem_type = kv->at;
  if (n) *n = kv->an;
  if (data) *data = scalar_bytes(kv->at) ? (const void *)(g->map + kv->apos) : NULL;
  return 1;
}

int amdc_gguf_get_arr_str(const amdc_gguf *g, const char *key, uint64_t i, const char **p, uint64_t *n) {
  const kv_t *kv = find(g, key);
  if (!kv || kv->type != AMDC_GGUF_ARR || kv->at != AMDC_GGUF_STR || !kv->astr || i >= kv->an) return 0;
  u64 len;
  memcpy(&len, g->map + kv->astr[i], 8);
  if (p) *p = (const char *)g->map + kv->astr[i] + 8u;
  if (n) *n = len;
  return 1;
}

int amdc_gguf_tensor_at(const amdc_gguf *g, uint64_t i, amdc_gguf_tensor *out) {
  if (!g || !out || i >= g->n_t) return gfail(AMDC_EINVAL, "gguf_tensor_at: no tensor %llu", (unsigned long long)i);
  *out = g->t[i];
  return AMDC_OK;
}

int64_t amdc_gguf_find_tensor(const amdc_gguf *g, const char *name) {
  for (u64 i = 0; g && name && i < g->n_t; i++)
    if (strcmp(g->t[i].name, name) == 0) return (int64_t)i;
  return -1;
}

/* ---------------------------------------------------------------- matrices (host side) */

int amdc_gguf_mat_kind(uint32_t ggml_type) {
  switch (ggml_type) {
    case 2: return AMDC_KIND_Q4_0;
    case 8: return AMDC_KIND_Q8_0;
    case 12: return AMDC_KIND_Q4_K;
    case 14: return AMDC_KIND_Q6_K;
    default: return -1;
  }
}

int amdc_gguf_mat_info(const amdc_gguf *g, const char *name, amdc_mat *m) {
  if (!g || !name || !m) return gfail(AMDC_EINVAL, "gguf_mat_info: null argument");
  const int64_t i = amdc_gguf_find_tensor(g, name);
  if (i < 0) return gfail(AMDC_EINVAL, "gguf: no tensor %s", name);
  const amdc_gguf_tensor *t = &g->t[i];
  const int kind = amdc_gguf_mat_kind(t->type);
  if (kind < 0) return gfail(AMDC_EINVAL, "gguf: tensor %s has GGML type %u, not one of Q4_0, Q8_0, Q4_K, Q6_K", name, t->type);
  if (t->ne[2] != 1u || t->ne[3] != 1u || t->ne[0] > 0xFFFFFFFFu || t->ne[1] > 0xFFFFFFFFu || !t->ne[0] || !t->ne[1])
    return gfail(AMDC_EINVAL, "gguf: tensor %s is not a matrix of 32-bit sizes", name);
  const u32 cols = (u32)t->ne[0], rows = (u32)t->ne[1];
  const u64 bytes = amdc_mat_bytes(kind, rows, cols);
  if (!bytes || !t->data) return gfail(AMDC_EINVAL, "gguf: tensor %s: %u x %u does not fit its kind", name, rows, cols);
  memset(m, 0, sizeof *m);
  m->kind = kind, m->rows = rows, m->cols = cols, m->nb = cols / 32u, m->bytes = bytes;
  return AMDC_OK;
}

typedef int (*repack_fn)(const uint8_t *, uint32_t, uint32_t, uint8_t *);

static repack_fn repack_of(int kind) {
  return kind == AMDC_KIND_Q4_0 ? amdc_repack_q4 : kind == AMDC_KIND_Q8_0 ? amdc_repack_q8 : kind == AMDC_KIND_Q4_K ? amdc_repack_q4k
                                                                                                                  : amdc_repack_q6k;
}

typedef struct {
  repack_fn f;
  const uint8_t *src; /* the job's first source row */
  uint8_t *dst;       /* the job's first destination row */
  u32 n, cols;        /* rows of the job */
  int rc;
} rjob;

static void *rjob_run(void *p) {
  rjob *j = p;
  j->rc = j->n ? j->f(j->src, j->n, j->cols, j->dst) : AMDC_OK;
  return NULL;
}

/* rows [r0, r1) of tensor t (kind m->kind) into dst (the rows' destination,
 * row r0 at dst) over nthreads threads */
AMDC_HIDDEN int amdc_gguf_repack_rows(const amdc_gguf_tensor *t, const amdc_mat *m, u32 r0, u32 r1, int nthreads, uint8_t *dst) {
  const u64 sb = amdc_ggml_nbytes(t->type, m->cols), db = m->bytes / m->rows;
  int nt = nthreads > 0 ? nthreads : (int)(((u64)(r1 - r0) * sb) / (1u << 20)) + 1;
  if (nt > 16) nt = 16;
  if ((u32)nt > r1 - r0) nt = (int)(r1 - r0);
  if (nt < 1) nt = 1;
  rjob jobs[16];
  pthread_t th[16];
  int started[16] = {0};
  for (int k = 0; k < nt; k++) {
    const u32 a = r0 + (u32)((u64)(r1 - r0) * (u64)k / (u64)nt), b = r0 + (u32)((u64)(r1 - r0) * (u64)(k + 1) / (u64)nt);
    jobs[k] = (rjob){repack_of(m->kind), (const uint8_t *)t->data + (u64)a * sb, dst + (u64)(a - r0) * db, b - a, m->cols, AMDC_OK};
    if (k > 0) started[k] = pthread_create(&th[k], NULL, rjob_run, &jobs[k]) == 0;
  }
  rjob_run(&jobs[0]);
  int rc = jobs[0].rc;
  for (int k = 1; k < nt; k++) {
    if (started[k]) pthread_join(th[k], NULL);
    else rjob_run(&jobs[k]); /* no thread: do it here */
    if (!rc) rc = jobs[k].rc;
  }
  return rc;
}

AMDC_HIDDEN int amdc_gguf_tensor_ptr(const amdc_gguf *g, const char *name, const amdc_gguf_tensor **t) {
  const int64_t i = amdc_gguf_find_tensor(g, name);
  if (i < 0) return gfail(AMDC_EINVAL, "gguf: no tensor %s", name);
  *t = &g->t[i];
  return AMDC_OK;
}

int amdc_gguf_repack(const amdc_gguf *g, const char *name, int nthreads, amdc_mat *m, uint8_t *dst) {
  if (!dst) return gfail(AMDC_EINVAL, "gguf_repack: null destination");
  int rc = amdc_gguf_mat_info(g, name, m);
  const amdc_gguf_tensor *t = NULL;
  if (!rc) rc = amdc_gguf_tensor_ptr(g, name, &t);
  return rc ? rc : amdc_gguf_repack_rows(t, m, 0, m->rows, nthreads, dst);
}
