/* launch_op.c -- the reference host's dispatch, written against include/amdc_q4.h and built
 * with gcc alone: the way hanw/amd.c's src/hip.c would drive libamdc_q4.so.
 *
 * It mirrors the reference's pieces for this path:
 *  - the arena: one device allocation; every buffer at a 256-byte aligned offset, one row per
 *    token at a 256-byte aligned stride (src/model.c:1194, the TP() macro of launch_op,
 *    src/hip.c:889);
 *  - a graph of two ops, OP_QUANT (x -> q) then OP_GEMV_<kind> (q -> y, + bias, + res), run
 *    over T tokens by one launch_op call each (src/hip.c:922-1089) on the engine's cur_stream;
 *  - IE_GEMM_MIN is left to the environment, read by the library as the reference reads it
 *    (src/hip.c:972-974);
 *  - errors: print and exit(1) (ie_die, src/common.c:6-14).
 * The run is eager once, then captured into a HIP graph and replayed three times; every replay
 * must give the eager bits.
 *
 * Usage: launch_op <kind> <rows> <cols> <T> <dir>
 *   dir/w.gguf   the GGUF bytes of the rows x cols matrix (AMDC_KIND_* kind)
 *   dir/x.f32    T x cols floats
 *   dir/bias.f32 rows floats (optional), dir/res.f32 T x rows floats (optional)
 * writes dir/q8.bin (T x 40 nb bytes: each token's Q8 buffer) and dir/y.f32 (T x rows). */
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "amdc_q4.h"

typedef uint32_t u32;

static void ie_die(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  fputs("launch_op: ", stderr);
  vfprintf(stderr, fmt, ap);
  fputc('\n', stderr);
  va_end(ap);
  exit(1);
}

static void *read_file(const char *dir, const char *name, size_t want, int optional) {
  char path[4096];
  snprintf(path, sizeof path, "%s/%s", dir, name);
  FILE *f = fopen(path, "rb");
  if (!f) {
    if (optional) return NULL;
    ie_die("cannot open %s", path);
  }
  void *p = malloc(want ? want : 1);
  if (!p || fread(p, 1, want, f) != want || fgetc(f) != EOF) ie_die("%s: expected exactly %zu bytes", path, want);
  fclose(f);
  return p;
}

static void write_file(const char *dir, const char *name, const void *p, size_t n) {
  char path[4096];
  snprintf(path, sizeof path, "%s/%s", dir, name);
  FILE *f = fopen(path, "wb");
  if (!f || fwrite(p, 1, n, f) != n || fclose(f)) ie_die("cannot write %s", path);
}

/* ---------------------------------------------------------------- the engine's graph */

enum { OP_QUANT, OP_GEMV };
typedef struct {
  size_t off;
  u32 stride; /* bytes per token */
} buf;
typedef struct {
  int kind; /* AMDC_KIND_*: the reference's MAT_* values */
  u32 rows, nb;
  void *d0;          /* the repacked matrix on the device */
  const float *bias; /* device, rows floats, or NULL */
} mat;
typedef struct {
  int kind, a, b, res; /* buffer ids, -1: none */
  u32 n;
  const mat *w;
} op;
typedef struct {
  buf bufs[4];
  op ops[2];
  int n_ops;
  unsigned char *arena;
  void *cur_stream;
} engine;

static u32 align256(size_t n) { return (u32)((n + 255u) & ~(size_t)255u); }

/* One op over T tokens, as launch_op (src/hip.c:882-1089) with the library in place of its
 * kernels. */
static void launch_op(engine *e, int i, u32 T) {
  const op *o = &e->ops[i];
#define TP(id) ((id) >= 0 ? (void *)(e->arena + e->bufs[id].off) : NULL)
  void *A = TP(o->a), *B = TP(o->b), *R = TP(o->res);
#undef TP
  switch (o->kind) {
    case OP_QUANT: {
      u32 nb = o->n / 32u, xs = e->bufs[o->a].stride, qs = e->bufs[o->b].stride;
      if (amdc_quant_q8(A, B, nb, T, xs, qs, e->cur_stream)) ie_die("%s", amdc_last_error());
      break;
    }
    case OP_GEMV: {
      const mat *w = o->w;
      u32 xs = e->bufs[o->a].stride, ys = e->bufs[o->b].stride / 4u, rs = o->res >= 0 ? e->bufs[o->res].stride / 4u : 0u;
      if (amdc_op_gemv(w->kind, w->d0, A, B, w->rows, w->nb, w->bias, R, T, xs, ys, rs, e->cur_stream))
        ie_die("%s", amdc_last_error());
      break;
    }
  }
}

static void run_ops(engine *e, u32 T) {
  for (int i = 0; i < e->n_ops; i++) launch_op(e, i, T);
}

int main(int argc, char **argv) {
  if (argc != 6) ie_die("usage: launch_op <kind> <rows> <cols> <T> <dir>");
  const int kind = atoi(argv[1]);
  const u32 rows = (u32)strtoul(argv[2], NULL, 10), cols = (u32)strtoul(argv[3], NULL, 10), T = (u32)strtoul(argv[4], NULL, 10);
  const char *dir = argv[5];
  const u32 nb = cols / 32u;
  const size_t gb = kind == AMDC_KIND_Q4_0 ? 18u * nb : kind == AMDC_KIND_Q8_0 ? 34u * nb
                    : kind == AMDC_KIND_Q4_K ? 144u * (cols / 256u) : 210u * (cols / 256u);
  if (!rows || !nb || !T || cols % 32u) ie_die("bad shape");

  if (amdc_open(NULL)) ie_die("gpu: %s", amdc_last_error());

  /* load time: repack on the host, upload (load_mat_src + gpu_sink) */
  unsigned char *gguf = read_file(dir, "w.gguf", gb * rows, 0);
  const size_t wbytes = amdc_mat_bytes(kind, rows, cols);
  if (!wbytes) ie_die("unsupported kind %d or shape %ux%u", kind, rows, cols);
  unsigned char *packed = malloc(wbytes);
  int rc = kind == AMDC_KIND_Q4_0   ? amdc_repack_q4(gguf, rows, cols, packed)
           : kind == AMDC_KIND_Q4_K ? amdc_repack_q4k(gguf, rows, cols, packed)
           : kind == AMDC_KIND_Q8_0 ? amdc_repack_q8(gguf, rows, cols, packed)
                                    : amdc_repack_q6k(gguf, rows, cols, packed);
  if (rc) ie_die("%s", amdc_last_error());
  mat w = {kind, rows, nb, NULL, NULL};
  if (amdc_malloc(&w.d0, wbytes) || amdc_memcpy_h2d(w.d0, packed, wbytes)) ie_die("%s", amdc_last_error());
  float *bias = read_file(dir, "bias.f32", (size_t)rows * 4u, 1);
  float *res = read_file(dir, "res.f32", (size_t)T * rows * 4u, 1);
  float *x = read_file(dir, "x.f32", (size_t)T * cols * 4u, 0);
  void *dbias = NULL;
  if (bias && (amdc_malloc(&dbias, (size_t)rows * 4u) || amdc_memcpy_h2d(dbias, bias, (size_t)rows * 4u)))
    ie_die("%s", amdc_last_error());
  w.bias = dbias;

  /* the arena: x, q, y, res; offsets and token strides 256-byte aligned */
  engine e = {0};
  enum { BX, BQ, BY, BR };
  const u32 strides[4] = {align256((size_t)cols * 4u), align256((size_t)nb * 40u), align256((size_t)rows * 4u),
                          align256((size_t)rows * 4u)};
  size_t off = 0;
  for (int b = 0; b < 4; b++) {
    e.bufs[b].off = off;
    e.bufs[b].stride = strides[b];
    off += (size_t)strides[b] * T;
  }
  if (amdc_malloc((void **)&e.arena, off) || amdc_memset(e.arena, 0xFF, off)) ie_die("%s", amdc_last_error());
  for (u32 t = 0; t < T; t++) {
    if (amdc_memcpy_h2d(e.arena + e.bufs[BX].off + (size_t)t * strides[BX], x + (size_t)t * cols, (size_t)cols * 4u))
      ie_die("%s", amdc_last_error());
    if (res && amdc_memcpy_h2d(e.arena + e.bufs[BR].off + (size_t)t * strides[BR], res + (size_t)t * rows, (size_t)rows * 4u))
      ie_die("%s", amdc_last_error());
  }
  e.ops[0] = (op){OP_QUANT, BX, BQ, -1, cols, NULL};
  e.ops[1] = (op){OP_GEMV, BQ, BY, res ? BR : -1, cols, &w};
  e.n_ops = 2;
  if (amdc_stream_create(&e.cur_stream)) ie_die("%s", amdc_last_error());

  /* eager */
  run_ops(&e, T);
  if (amdc_stream_sync(e.cur_stream)) ie_die("%s", amdc_last_error());
  unsigned char *q8 = malloc((size_t)T * nb * 40u);
  float *y = malloc((size_t)T * rows * 4u), *yg = malloc((size_t)T * rows * 4u);
  for (u32 t = 0; t < T; t++) {
    if (amdc_memcpy_d2h(q8 + (size_t)t * nb * 40u, e.arena + e.bufs[BQ].off + (size_t)t * strides[BQ], (size_t)nb * 40u) ||
        amdc_memcpy_d2h(y + (size_t)t * rows, e.arena + e.bufs[BY].off + (size_t)t * strides[BY], (size_t)rows * 4u))
      ie_die("%s", amdc_last_error());
  }

  /* the same ops captured once, replayed three times */
  void *exec = NULL;
  if (amdc_graph_begin(e.cur_stream)) ie_die("%s", amdc_last_error());
  run_ops(&e, T);
  if (amdc_graph_end(e.cur_stream, &exec)) ie_die("%s", amdc_last_error());
  for (int r = 0; r < 3; r++) {
    if (amdc_memset(e.arena + e.bufs[BQ].off, 0xFF, (size_t)strides[BQ] * T) ||
        amdc_memset(e.arena + e.bufs[BY].off, 0xFF, (size_t)strides[BY] * T))
      ie_die("%s", amdc_last_error());
    if (amdc_graph_launch(exec, e.cur_stream) || amdc_stream_sync(e.cur_stream)) ie_die("%s", amdc_last_error());
    for (u32 t = 0; t < T; t++) {
      if (amdc_memcpy_d2h(yg + (size_t)t * rows, e.arena + e.bufs[BY].off + (size_t)t * strides[BY], (size_t)rows * 4u))
        ie_die("%s", amdc_last_error());
    }
    if (memcmp(y, yg, (size_t)T * rows * 4u)) ie_die("graph replay %d differs from the eager run", r);
  }
  write_file(dir, "q8.bin", q8, (size_t)T * nb * 40u);
  write_file(dir, "y.f32", y, (size_t)T * rows * 4u);
  printf("launch_op: kind %d %ux%u T=%u ok\n", kind, rows, cols, T);

  amdc_graph_destroy(exec);
  amdc_stream_destroy(e.cur_stream);
  amdc_free(e.arena);
  amdc_free(w.d0);
  if (dbias) amdc_free(dbias);
  amdc_close();
  free(gguf), free(packed), free(bias), free(res), free(x), free(q8), free(y), free(yg);
  return 0;
}
