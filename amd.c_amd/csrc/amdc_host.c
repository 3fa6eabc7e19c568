/* amdc_host.c -- the C host of the MI355X quantized GEMV/GEMM path
 * (libamdc_q4.so; the ABI is include/amdc_q4.h).
 *
 * As the reference's GPU host (hanw/amd.c src/hip.c), it needs no ROCm
 * headers: the HIP runtime is dlopen'ed and the kernels are resolved by name
 * from a code object (amdc_kernels.hsaco) and launched with
 * hipModuleLaunchKernel and a void* argument array. It also holds the
 * load-time repack into the CDNA4 layout (amdc_layout.h), which replaces
 * repack_q4 / repack_q4k of src/model.c. */
#define _GNU_SOURCE
#include "../../include/amdc_q4.h"
#include "../../include/amdc_gguf.h"

#include <dlfcn.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "amdc_internal.h"
#include "amdc_layout.h"

typedef uint32_t u32;
typedef uint64_t u64;

/* ---------------------------------------------------------------- errors */

static char g_err[512];

int amdc_fail_v(int code, const char *fmt, va_list ap) {
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  return code;
}

static int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  amdc_fail_v(code, fmt, ap);
  va_end(ap);
  return code;
}

const char *amdc_last_error(void) { return g_err; }

/* ---------------------------------------------------------------- repack */

static int kind_ok(int kind) {
  return kind == AMDC_KIND_Q4_0 || kind == AMDC_KIND_Q4_K || kind == AMDC_KIND_Q8_0 || kind == AMDC_KIND_Q6_K;
}

size_t amdc_mat_bytes(int kind, uint32_t rows, uint32_t cols) {
  if (cols % 32u || ((kind == AMDC_KIND_Q4_K || kind == AMDC_KIND_Q6_K) && cols % 256u) || !kind_ok(kind)) return 0;
  return (size_t)rows * amdc_row_bytes_k(kind, cols / 32u);
}

/* GGUF Q4_0: block b of row r = 18 bytes at (r nb + b) 18: f16 d, then
 * nibble byte j (weight j low, j + 16 high). The 16 nibble bytes go to the
 * block's slot unchanged, d to its header (src/model.c:205-219 keeps the same
 * bytes in another order). */
int amdc_repack_q4(const uint8_t *src, uint32_t rows, uint32_t cols, uint8_t *dst) {
  if (!src || !dst || !rows || !cols || cols % 32u) return fail(AMDC_EINVAL, "repack_q4: %ux%u (cols must be a multiple of 32)", rows, cols);
  const u32 nb = cols / 32u, ng = amdc_ngroups(nb);
  const u64 rb = amdc_row_bytes(nb);
  memset(dst, 0, (size_t)rows * rb);
  for (u32 r = 0; r < rows; r++) {
    uint8_t *row = dst + (u64)r * rb;
    for (u32 b = 0; b < nb; b++) {
      const uint8_t *blk = src + ((u64)r * nb + b) * 18u;
      const u32 g = b >> 3, k = b & 7u;
      row[amdc_header_off(g) + 2u * k] = blk[0];
      row[amdc_header_off(g) + 2u * k + 1u] = blk[1];
      memcpy(row + amdc_nib_off(ng, g, k), blk + 2, 16);
    }
  }
  return AMDC_OK;
}

/* The 6-bit scale and min of sub-block j of a Q4_K super-block from its 12
 * scale bytes (ggml's get_scale_min_k4, as src/model.c:24-31). */
static void q4k_scale_min(u32 j, const uint8_t *s, u32 *sc, u32 *mn) {
  if (j < 4) {
    *sc = s[j] & 63u;
    *mn = s[j + 4] & 63u;
  } else {
    *sc = (s[j + 4] & 15u) | ((u32)(s[j - 4] >> 6) << 4);
    *mn = (u32)(s[j + 4] >> 4) | ((u32)(s[j] >> 6) << 4);
  }
}

/* GGUF Q4_K: super-block g of row r = 144 bytes: f16 d, f16 dmin, 12 scale
 * bytes, 128 nibble bytes (sub-blocks 2i and 2i+1 are the low and high
 * nibbles of bytes 32i..32i+31). Sub-block k becomes a Q4_0-order block (byte
 * j: weight j low, j + 16 high), as MAT_Q4K (src/model.c:246-267); the
 * header keeps d and dmin and packs sc_0..7 and mn_0..7 six bits each. */
int amdc_repack_q4k(const uint8_t *src, uint32_t rows, uint32_t cols, uint8_t *dst) {
  if (!src || !dst || !rows || !cols || cols % 256u)
    return fail(AMDC_EINVAL, "repack_q4k: %ux%u (cols must be a multiple of 256)", rows, cols);
  const u32 nb = cols / 32u, ng = nb / 8u;
  const u64 rb = amdc_row_bytes(nb);
  for (u32 r = 0; r < rows; r++) {
    uint8_t *row = dst + (u64)r * rb;
    for (u32 g = 0; g < ng; g++) {
      const uint8_t *blk = src + ((u64)r * ng + g) * 144u;
      uint8_t *hd = row + amdc_header_off(g);
      u64 scs = 0, mns = 0;
      for (u32 k = 0; k < 8; k++) {
        u32 sc, mn;
        q4k_scale_min(k, blk + 4, &sc, &mn);
        scs |= (u64)sc << (6u * k);
        mns |= (u64)mn << (6u * k);
      }
      memcpy(hd, blk, 4); /* f16 d, f16 dmin */
      for (u32 i = 0; i < 6; i++) hd[4 + i] = (uint8_t)(scs >> (8u * i)), hd[10 + i] = (uint8_t)(mns >> (8u * i));
      for (u32 k = 0; k < 8; k++) {
        const uint8_t *pair = blk + 16 + 32u * (k >> 1);
        uint8_t *o = row + amdc_nib_off(ng, g, k);
        for (u32 j = 0; j < 16; j++) {
          const u32 lo = (k & 1u) ? (u32)pair[j] >> 4 : pair[j] & 15u, hi = (k & 1u) ? (u32)pair[j + 16] >> 4 : pair[j + 16] & 15u;
          o[j] = (uint8_t)(lo | (hi << 4));
        }
      }
    }
  }
  return AMDC_OK;
}

/* GGUF Q8_0: block b of row r = 34 bytes at (r nb + b) 34: f16 d, 32 int8.
 * The int8 bytes go to planes 2k, 2k + 1 of the block's super-group, d to
 * its header (src/model.c:221-237 keeps the same bytes as 8 words per block
 * and a separate f16 array). */
int amdc_repack_q8(const uint8_t *src, uint32_t rows, uint32_t cols, uint8_t *dst) {
  if (!src || !dst || !rows || !cols || cols % 32u) return fail(AMDC_EINVAL, "repack_q8: %ux%u (cols must be a multiple of 32)", rows, cols);
  const u32 nb = cols / 32u, ng = amdc_ngroups(nb);
  const u64 rb = amdc_q8_row_bytes(nb);
  memset(dst, 0, (size_t)rows * rb);
  for (u32 r = 0; r < rows; r++) {
    uint8_t *row = dst + (u64)r * rb;
    for (u32 b = 0; b < nb; b++) {
      const uint8_t *blk = src + ((u64)r * nb + b) * 34u;
      const u32 g = b >> 3, k = b & 7u;
      memcpy(row + amdc_header_off(g) + 2u * k, blk, 2);
      memcpy(row + amdc_q8_off(ng, g, 2u * k), blk + 2, 16);
      memcpy(row + amdc_q8_off(ng, g, 2u * k + 1u), blk + 18, 16);
    }
  }
  return AMDC_OK;
}

/* GGUF Q6_K: super-block g of row r = 210 bytes: ql[128], qh[64], int8
 * scales[16], f16 d. Weight e = 128 n + 32 m + l has the low 4 bits of
 * ql[64 n + 32 (m & 1) + l] (low nibble for m < 2, else high) and the 2 bits
 * (qh[32 n + l] >> 2 m) & 3 above them (core/ie_core.h:309-313, 338-341).
 * Sub-block k (weights 32k..32k+31) becomes a Q4_0-order nibble block and two
 * high-bit words, as MAT_Q6K (src/model.c:269-292); scales and d are copied. */
int amdc_repack_q6k(const uint8_t *src, uint32_t rows, uint32_t cols, uint8_t *dst) {
  if (!src || !dst || !rows || !cols || cols % 256u)
    return fail(AMDC_EINVAL, "repack_q6k: %ux%u (cols must be a multiple of 256)", rows, cols);
  const u32 nb = cols / 32u, ng = nb / 8u;
  const u64 rb = amdc_q6k_row_bytes(nb);
  for (u32 r = 0; r < rows; r++) {
    uint8_t *row = dst + (u64)r * rb;
    memset(row + 16u * ng, 0, amdc_q6k_dpad(ng));
    for (u32 g = 0; g < ng; g++) {
      const uint8_t *blk = src + ((u64)r * ng + g) * 210u;
      memcpy(row + amdc_header_off(g), blk + 192, 16);
      memcpy(row + amdc_q6k_d_off(ng, g), blk + 208, 2);
      for (u32 k = 0; k < 8; k++) {
        const u32 n = k / 4u, m = k % 4u;
        u32 q[32];
        for (u32 l = 0; l < 32; l++) {
          const uint8_t lo = blk[64u * n + 32u * (m & 1u) + l];
          q[l] = (m < 2u ? (lo & 15u) : (u32)(lo >> 4)) | ((((u32)blk[128u + 32u * n + l] >> (2u * m)) & 3u) << 4);
        }
        uint8_t *o = row + amdc_q6k_nib_off(ng, g, k);
        for (u32 j = 0; j < 16; j++) o[j] = (uint8_t)((q[j] & 15u) | ((q[j + 16] & 15u) << 4));
        uint8_t *hp = row + amdc_q6k_hi_off(ng, g, k >> 1) + 8u * (k & 1u);
        for (u32 h = 0; h < 2; h++) {
          u32 wd = 0;
          for (u32 e = 0; e < 16; e++) wd |= (q[16u * h + e] >> 4) << (8u * (e % 4u) + 2u * (e / 4u));
          memcpy(hp + 4u * h, &wd, 4);
        }
      }
    }
  }
  return AMDC_OK;
}

/* ---------------------------------------------------------------- HIP through dlopen */

typedef int hipError_t;
typedef void *hipModule_t, *hipFunction_t, *hipStream_t, *hipEvent_t, *hipGraph_t, *hipGraphExec_t;
enum { hipStreamCaptureModeRelaxed = 2 };
enum { hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2, hipMemcpyDeviceToDevice = 3 };
enum { hipDeviceAttributeMultiprocessorCount = 63 };

static struct {
  void *lib;
  hipError_t (*GetDeviceCount)(int *);
  hipError_t (*SetDevice)(int);
  hipError_t (*DeviceGetAttribute)(int *, int, int);
  hipError_t (*ModuleLoad)(hipModule_t *, const char *);
  hipError_t (*ModuleUnload)(hipModule_t);
  hipError_t (*ModuleGetFunction)(hipFunction_t *, hipModule_t, const char *);
  hipError_t (*ModuleGetGlobal)(void **, size_t *, hipModule_t, const char *);
  hipError_t (*ModuleLaunchKernel)(hipFunction_t, unsigned, unsigned, unsigned, unsigned, unsigned, unsigned, unsigned, hipStream_t,
                                   void **, void **);
  hipError_t (*Malloc)(void **, size_t);
  hipError_t (*Free)(void *);
  hipError_t (*Memcpy)(void *, const void *, size_t, int);
  hipError_t (*Memset)(void *, int, size_t);
  hipError_t (*DeviceSynchronize)(void);
  hipError_t (*EventCreate)(hipEvent_t *);
  hipError_t (*EventDestroy)(hipEvent_t);
  hipError_t (*EventRecord)(hipEvent_t, hipStream_t);
  hipError_t (*EventSynchronize)(hipEvent_t);
  hipError_t (*EventElapsedTime)(float *, hipEvent_t, hipEvent_t);
  const char *(*GetErrorString)(hipError_t);
  hipError_t (*StreamCreate)(hipStream_t *);
  hipError_t (*StreamDestroy)(hipStream_t);
  hipError_t (*StreamSynchronize)(hipStream_t);
  hipError_t (*StreamWaitEvent)(hipStream_t, hipEvent_t, unsigned);
  hipError_t (*StreamBeginCapture)(hipStream_t, int);
  hipError_t (*StreamEndCapture)(hipStream_t, hipGraph_t *);
  hipError_t (*GraphInstantiate)(hipGraphExec_t *, hipGraph_t, void *, char *, size_t);
  hipError_t (*GraphDestroy)(hipGraph_t);
  hipError_t (*GraphLaunch)(hipGraphExec_t, hipStream_t);
  hipError_t (*GraphExecDestroy)(hipGraphExec_t);
  hipError_t (*OccupancyMaxActiveBlocks)(int *, hipFunction_t, int, size_t);
  hipError_t (*HostMalloc)(void **, size_t, unsigned);
  hipError_t (*HostFree)(void *);
  hipError_t (*MemcpyAsync)(void *, const void *, size_t, int, hipStream_t);
} H;

/* The kernels of amdc_kernels.hip. */
enum {
  K_QUANT,
  K_DOTS_Q4,
  K_DOTS_Q4K,
  K_GEMM_N128,
  K_GEMM_N64,
  K_GEMV_Q4_P1,
  K_GEMV_Q4K_P1,
  K_PROBE_READ,
  K_PROBE_COPY,
  K_Q8_PREP,
  K_GEMMH_M64_N128,
  K_GEMMH_M64_N64,
  K_GEMM_REDUCE,
  K_GEMV_Q4_V8,
  K_GEMV_Q4K_V8,
  K_GEMV_Q4_X1,
  K_GEMV_Q4K_X1,
  K_GEMV_Q4_P2,
  K_GEMV_Q4K_P2,
  K_CHAIN,
  K_RMSNORM_Q8,
  K_SWIGLU_Q8,
  K_GEMV_Q8_P2,
  K_GEMV_Q6K_P2,
  K_DOTS_Q8,
  K_DOTS_Q6K,
  K_GEMMH_Q8_N128,
  K_GEMMH_Q8_N64,
  K_GEMMH_Q6K_N128,
  K_GEMMH_Q6K_N64,
  K_GEMV_Q8_V8,
  K_GEMV_Q6K_V8,
  K_GEMMH_Q4_N128,
  K_GEMMH_Q4_N64,
  K_GEMV_Q4_V16,
  K_GEMV_Q4K_V16,
  K_GEMV_Q8_V16,
  K_GEMV_Q6K_V16,
  K_GEMVS_Q4, /* amdc_gemv_q4_0_s1 .. _s4, then amdc_gemv_q4_k_s1 .. _s4 */
  K_GEMVXS_Q4 = K_GEMVS_Q4 + 8, /* amdc_gemv_q4_0_xs1 .. _xs4, then amdc_gemv_q4_k_xs1 .. _xs4 */
  K_GEMVM_Q4 = K_GEMVXS_Q4 + 8, /* amdc_gemv_q4_0_m1, amdc_gemv_q4_k_m1 */
  K_CHAIN_S = K_GEMVM_Q4 + 2, /* amdc_chain_s_q4_0, amdc_chain_s_q4_k */
  K_GEMVXW_Q4 = K_CHAIN_S + 2, /* amdc_gemv_q4_0_xw1, amdc_gemv_q4_k_xw1, _xw2 */
  K_GEMVK_Q4 = K_GEMVXW_Q4 + 3, /* amdc_gemv_q4_0_k, _xk, amdc_gemv_q4_k_k, _xk */
  K_GEMVSN_Q4 = K_GEMVK_Q4 + 4, /* amdc_gemv_q4_0_n1 .. _n4, amdc_gemv_q4_k_n1 .. _n4 (fused RMSNorm tail) */
  K_GEMV2N = K_GEMVSN_Q4 + 8,   /* amdc_gemv_q8_0_pn, _q6_k_pn */
  K_GEMMH_M128 = K_GEMV2N + 2,  /* amdc_gemmh_m128_n128 */
  K_GEMVM8 = K_GEMMH_M128 + 1,  /* amdc_gemv_q8_0_m1, amdc_gemv_q6_k_m1 */
  K_GEMVS1W = K_GEMVM8 + 2,     /* amdc_gemv_q4_0_s1w, amdc_gemv_q4_k_s1w */
  K_N = K_GEMVS1W + 2
};
static const char *const kname[K_N] = {
    "amdc_quant_q8",           "amdc_dots_q4_0",          "amdc_dots_q4_k",          "amdc_gemm_q4_k_n128",
    "amdc_gemm_q4_k_n64",      "amdc_gemv_q4_0_p1",       "amdc_gemv_q4_k_p1",       "amdc_probe_read",
    "amdc_probe_copy",         "amdc_q8_prep",            "amdc_gemmh_m64_n128",     "amdc_gemmh_m64_n64",
    "amdc_gemm_reduce",        "amdc_gemv_q4_0_v8",       "amdc_gemv_q4_k_v8",       "amdc_gemv_q4_0_x1",
    "amdc_gemv_q4_k_x1",       "amdc_gemv_q4_0_p2",       "amdc_gemv_q4_k_p2",       "amdc_chain",
    "amdc_rmsnorm_q8",         "amdc_swiglu_q8",          "amdc_gemv_q8_0_p2",       "amdc_gemv_q6_k_p2",
    "amdc_dots_q8_0",          "amdc_dots_q6_k",          "amdc_gemmh_q8_0_m64_n128", "amdc_gemmh_q8_0_m64_n64",
    "amdc_gemmh_q6_k_m64_n128", "amdc_gemmh_q6_k_m64_n64", "amdc_gemv_q8_0_v8",       "amdc_gemv_q6_k_v8",
    "amdc_gemmh_q4_0_m64_n128", "amdc_gemmh_q4_0_m64_n64", "amdc_gemv_q4_0_v16",      "amdc_gemv_q4_k_v16",
    "amdc_gemv_q8_0_v16",      "amdc_gemv_q6_k_v16",
    "amdc_gemv_q4_0_s1",       "amdc_gemv_q4_0_s2",       "amdc_gemv_q4_0_s3",       "amdc_gemv_q4_0_s4",
    "amdc_gemv_q4_k_s1",       "amdc_gemv_q4_k_s2",       "amdc_gemv_q4_k_s3",       "amdc_gemv_q4_k_s4",
    "amdc_gemv_q4_0_xs1",      "amdc_gemv_q4_0_xs2",      "amdc_gemv_q4_0_xs3",      "amdc_gemv_q4_0_xs4",
    "amdc_gemv_q4_k_xs1",      "amdc_gemv_q4_k_xs2",      "amdc_gemv_q4_k_xs3",      "amdc_gemv_q4_k_xs4",
    "amdc_gemv_q4_0_m1",       "amdc_gemv_q4_k_m1",       "amdc_chain_s_q4_0",       "amdc_chain_s_q4_k",
    "amdc_gemv_q4_0_xw1",      "amdc_gemv_q4_k_xw1",      "amdc_gemv_q4_k_xw2",      "amdc_gemv_q4_0_k",
    "amdc_gemv_q4_0_xk",       "amdc_gemv_q4_k_k",        "amdc_gemv_q4_k_xk",
    "amdc_gemv_q4_0_n1",       "amdc_gemv_q4_0_n2",       "amdc_gemv_q4_0_n3",       "amdc_gemv_q4_0_n4",
    "amdc_gemv_q4_k_n1",       "amdc_gemv_q4_k_n2",       "amdc_gemv_q4_k_n3",       "amdc_gemv_q4_k_n4",
    "amdc_gemv_q8_0_pn",       "amdc_gemv_q6_k_pn",       "amdc_gemmh_m128_n128",
    "amdc_gemv_q8_0_m1",       "amdc_gemv_q6_k_m1",       "amdc_gemv_q4_0_s1w",      "amdc_gemv_q4_k_s1w"};

static hipModule_t g_mod;
static hipFunction_t g_k[K_N];
static int g_occ[K_N]; /* resident workgroups per CU, looked up at a kernel's first use (0: not yet) */
static int g_open, g_cus;
static int t_lanes = -1, t_unroll = -1, t_wgs = -1, t_gemm = -1, t_gemm_min = -1, t_ksplit = -1;
static u32 *g_norm_cnt; /* the fused-norm GEMVs' arrival counter (device, 0 between launches) */
/* The largest T x rows x super-groups that runs on the few-vector Q8_0 / Q6_K kernels (tuning: AMDC_GEMVM8_MAX) */
static u64 M8_MAX = 786432u;
static u32 x_fuse_nb = 128; /* amdc_gemv_q4_x / _q4k_x: the largest nb quantized inside the GEMV */
/* The chain recorder (amdc_chain_record_begin / _end): while it is on, the recordable operators
 * called on its stream append chain operations instead of launching; every other launch on that
 * stream is refused. */
static struct {
  int on;
  void *stream;
  amdc_chain_op *ops;
  u32 n, cap, seg0;
  int err; /* an operator refused while recording: record_end reports it */
} g_rec;
static int t_form = 0;      /* decode GEMV: 1 = amdc_gemv_*_p1, 2 = amdc_gemv_*_p2, 0 = by shape */
/* The GEMM's device workspace (prepared activations, split-K partial sums): grown on demand;
 * the smaller ones it replaced stay allocated until amdc_close (see ws_reserve). */
static void *g_ws;
static size_t g_ws_bytes;
static void *g_ws_old[48];
static unsigned g_ws_old_n;
/* The code object's fixed workspace, the device array `scratch` of amdc_kernels.hip: its device
 * address and size, looked up once at amdc_open (the library drives device 0 only). Inside
 * amdc_op_gemv_noalloc (g_ws_fixed set) every workspace request is served from it, and a request
 * larger than it is an error; otherwise it is unused. */
static void *g_scratch;
static u32 *g_split_cnt; /* the kernels' split_count array (device address) */
static size_t g_scratch_bytes;
static int g_ws_fixed;

#define HIPCALL(x)                                                                               \
  do {                                                                                           \
    const hipError_t e_ = (x);                                                                   \
    if (e_) return fail(AMDC_EHIP, "%s: %s (%d)", #x, H.GetErrorString ? H.GetErrorString(e_) : "?", e_); \
  } while (0)
#define NEED_OPEN()                                                               \
  do {                                                                            \
    if (!g_open) return fail(AMDC_ENOTOPEN, "amdc_open has not been called"); \
  } while (0)

static int envi(const char *n, int dflt) {
  const char *v = getenv(n);
  return v && *v ? atoi(v) : dflt;
}

static int hip_load(void) {
  if (H.lib) return AMDC_OK;
  const char *names[] = {"libamdhip64.so.7", "libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"};
  for (unsigned i = 0; i < sizeof names / sizeof names[0] && !H.lib; i++) H.lib = dlopen(names[i], RTLD_NOW | RTLD_GLOBAL);
  if (!H.lib) return fail(AMDC_ENOHIP, "cannot load the HIP runtime (libamdhip64.so): %s", dlerror());
#define SYM(f, n)                                                                    \
  do {                                                                               \
    *(void **)&H.f = dlsym(H.lib, n);                                                \
    if (!H.f) return fail(AMDC_ENOHIP, "HIP runtime without %s", n);             \
  } while (0)
  SYM(GetDeviceCount, "hipGetDeviceCount");
  SYM(SetDevice, "hipSetDevice");
  SYM(DeviceGetAttribute, "hipDeviceGetAttribute");
  SYM(ModuleLoad, "hipModuleLoad");
  SYM(ModuleUnload, "hipModuleUnload");
  SYM(ModuleGetFunction, "hipModuleGetFunction");
  SYM(ModuleGetGlobal, "hipModuleGetGlobal");
  SYM(ModuleLaunchKernel, "hipModuleLaunchKernel");
  SYM(Malloc, "hipMalloc");
  SYM(Free, "hipFree");
  SYM(Memcpy, "hipMemcpy");
  SYM(Memset, "hipMemset");
  SYM(DeviceSynchronize, "hipDeviceSynchronize");
  SYM(EventCreate, "hipEventCreate");
  SYM(EventDestroy, "hipEventDestroy");
  SYM(EventRecord, "hipEventRecord");
  SYM(EventSynchronize, "hipEventSynchronize");
  SYM(EventElapsedTime, "hipEventElapsedTime");
  SYM(GetErrorString, "hipGetErrorString");
  SYM(StreamCreate, "hipStreamCreate");
  SYM(StreamDestroy, "hipStreamDestroy");
  SYM(StreamSynchronize, "hipStreamSynchronize");
  SYM(StreamWaitEvent, "hipStreamWaitEvent");
  SYM(StreamBeginCapture, "hipStreamBeginCapture");
  SYM(StreamEndCapture, "hipStreamEndCapture");
  SYM(GraphInstantiate, "hipGraphInstantiate");
  SYM(GraphDestroy, "hipGraphDestroy");
  SYM(GraphLaunch, "hipGraphLaunch");
  SYM(GraphExecDestroy, "hipGraphExecDestroy");
  SYM(OccupancyMaxActiveBlocks, "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor");
  SYM(HostMalloc, "hipHostMalloc");
  SYM(HostFree, "hipHostFree");
  SYM(MemcpyAsync, "hipMemcpyAsync");
#undef SYM
  return AMDC_OK;
}

int amdc_open(const char *hsaco) {
  if (g_open) return AMDC_OK;
  int rc = hip_load();
  if (rc) return rc;
  int n = 0;
  if (H.GetDeviceCount(&n) || n < 1) return fail(AMDC_ENOHIP, "no HIP device");
  HIPCALL(H.SetDevice(0));
  char path[4096];
  if (!hsaco) { /* next to this library */
    Dl_info di;
    if (!dladdr((void *)amdc_open, &di) || !di.dli_fname) return fail(AMDC_EINVAL, "cannot locate libamdc_q4.so");
    snprintf(path, sizeof path, "%s", di.dli_fname);
    char *s = strrchr(path, '/');
    if (s) s[1] = 0;
    else path[0] = 0;
    strncat(path, "amdc_kernels.hsaco", sizeof path - strlen(path) - 1);
    hsaco = path;
  }
  HIPCALL(H.ModuleLoad(&g_mod, hsaco));
  for (int k = 0; k < K_N; k++) HIPCALL(H.ModuleGetFunction(&g_k[k], g_mod, kname[k]));
  memset(g_occ, 0, sizeof g_occ);
  /* the module-API lookup of a device variable (hipGetSymbolAddress of a code object loaded with
     hipModuleLoad); with device 0 current. Host code uses this address, never the name. */
  HIPCALL(H.ModuleGetGlobal(&g_scratch, &g_scratch_bytes, g_mod, "scratch"));
  if (!g_scratch || g_scratch_bytes < AMDC_SCRATCH_BYTES)
    return fail(AMDC_EHIP, "amdc_kernels.hsaco: scratch array of %zu bytes, expected %zu", g_scratch_bytes, (size_t)AMDC_SCRATCH_BYTES);
  {
    size_t cb = 0;
    HIPCALL(H.ModuleGetGlobal((void **)&g_split_cnt, &cb, g_mod, "split_count"));
    if (!g_split_cnt || cb < AMDC_SPLIT_TILES * sizeof(u32))
      return fail(AMDC_EHIP, "amdc_kernels.hsaco: split_count array of %zu bytes, expected %zu", cb, AMDC_SPLIT_TILES * sizeof(u32));
    HIPCALL(H.Memset(g_split_cnt, 0, AMDC_SPLIT_TILES * sizeof(u32))); /* each launch leaves them at 0 again */
    HIPCALL(H.ModuleGetGlobal((void **)&g_norm_cnt, &cb, g_mod, "norm_count"));
    if (!g_norm_cnt || cb < sizeof(u32)) return fail(AMDC_EHIP, "amdc_kernels.hsaco: no norm_count counter");
    HIPCALL(H.Memset(g_norm_cnt, 0, cb));
  }
  HIPCALL(H.DeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, 0));
  if (t_lanes < 0) t_lanes = envi("AMDC_GEMV_L", 0);
  if (t_unroll < 0) t_unroll = envi("AMDC_GEMV_U", 0);
  if (t_wgs < 0) t_wgs = envi("AMDC_GEMV_WG", 0);
  if (t_gemm < 0) t_gemm = envi("AMDC_GEMM_KERNEL", 0);
  if (t_ksplit < 0) t_ksplit = envi("AMDC_GEMM_KSPLIT", 0);
  /* the token count from which op_gemv runs the prefill GEMM: the reference's IE_GEMM_MIN
     variable when set; else 0, the MI355X rule of use_gemm */
  if (t_gemm_min < 0) t_gemm_min = envi("IE_GEMM_MIN", 0);
  x_fuse_nb = (u32)envi("AMDC_GEMVX_FUSE_NB", 128);
  M8_MAX = (u64)envi("AMDC_GEMVM8_MAX", 786432);
  t_form = envi("AMDC_GEMV_FORM", 0);
  g_open = 1;
  return AMDC_OK;
}

static void stage_free(void);

void amdc_close(void) {
  free(g_rec.ops);
  memset(&g_rec, 0, sizeof g_rec);
  if (g_open) stage_free();
  if (g_open && g_ws) H.Free(g_ws);
  for (unsigned i = 0; g_open && i < g_ws_old_n; i++) H.Free(g_ws_old[i]);
  g_ws = NULL, g_ws_bytes = 0, g_ws_old_n = 0;
  g_scratch = NULL, g_scratch_bytes = 0, g_split_cnt = NULL;
  if (g_open && g_mod) H.ModuleUnload(g_mod);
  g_mod = NULL;
  g_open = 0;
}

int amdc_cu_count(void) { return g_open ? g_cus : 0; }

int amdc_set_tuning(int gemv_lanes, int gemv_unroll, int gemv_wgs, int gemm_kernel, int gemm_ksplit, int gemv_form) {
  if (gemv_lanes && (gemv_lanes < 4 || gemv_lanes > 64 || (gemv_lanes & (gemv_lanes - 1))))
    return fail(AMDC_EINVAL, "gemv lanes %d: 4..64, a power of two", gemv_lanes);
  if (gemv_unroll < 0 || gemv_unroll > 2) return fail(AMDC_EINVAL, "gemv unroll %d: 0, 1 or 2", gemv_unroll);
  if (gemm_kernel < 0 || gemm_kernel > 5) return fail(AMDC_EINVAL, "gemm kernel %d: 0..5", gemm_kernel);
  if (gemm_ksplit < 0 || gemm_ksplit > 16) return fail(AMDC_EINVAL, "gemm ksplit %d: 0..16", gemm_ksplit);
  if (gemv_wgs < 0) return fail(AMDC_EINVAL, "gemv workgroups %d", gemv_wgs);
  if (gemv_form < 0 || gemv_form > 4) return fail(AMDC_EINVAL, "gemv form %d: 0..4", gemv_form);
  t_lanes = gemv_lanes, t_unroll = gemv_unroll, t_wgs = gemv_wgs, t_gemm = gemm_kernel, t_ksplit = gemm_ksplit, t_form = gemv_form;
  return AMDC_OK;
}

int amdc_malloc(void **p, size_t n) {
  NEED_OPEN();
  HIPCALL(H.Malloc(p, n ? n : 1));
  return AMDC_OK;
}
int amdc_free(void *p) {
  NEED_OPEN();
  if (p) HIPCALL(H.Free(p));
  return AMDC_OK;
}
int amdc_memcpy_h2d(void *d, const void *s, size_t n) {
  NEED_OPEN();
  HIPCALL(H.Memcpy(d, s, n, hipMemcpyHostToDevice));
  return AMDC_OK;
}
int amdc_memcpy_d2h(void *d, const void *s, size_t n) {
  NEED_OPEN();
  HIPCALL(H.Memcpy(d, s, n, hipMemcpyDeviceToHost));
  return AMDC_OK;
}
int amdc_memcpy_d2d(void *d, const void *s, size_t n) {
  NEED_OPEN();
  HIPCALL(H.Memcpy(d, s, n, hipMemcpyDeviceToDevice));
  return AMDC_OK;
}
int amdc_memset(void *p, int v, size_t n) {
  NEED_OPEN();
  HIPCALL(H.Memset(p, v, n));
  return AMDC_OK;
}
int amdc_sync(void) {
  NEED_OPEN();
  HIPCALL(H.DeviceSynchronize());
  return AMDC_OK;
}
int amdc_event_create(void **ev) {
  NEED_OPEN();
  HIPCALL(H.EventCreate(ev));
  return AMDC_OK;
}
int amdc_event_destroy(void *ev) {
  NEED_OPEN();
  HIPCALL(H.EventDestroy(ev));
  return AMDC_OK;
}
int amdc_event_record(void *ev, void *stream) {
  NEED_OPEN();
  HIPCALL(H.EventRecord(ev, stream));
  return AMDC_OK;
}
int amdc_event_elapsed_ms(float *ms, void *a, void *b) {
  NEED_OPEN();
  HIPCALL(H.EventSynchronize(b));
  HIPCALL(H.EventElapsedTime(ms, a, b));
  return AMDC_OK;
}

/* Streams (default priority) and graphs: an op sequence captured once and
 * replayed, so that the GPU runs it without a host launch per kernel. The
 * operators record no memset, so their graphs hold kernel nodes only. */
int amdc_stream_create(void **s) {
  NEED_OPEN();
  HIPCALL(H.StreamCreate(s));
  return AMDC_OK;
}
int amdc_stream_destroy(void *s) {
  NEED_OPEN();
  HIPCALL(H.StreamDestroy(s));
  return AMDC_OK;
}
int amdc_stream_sync(void *s) {
  NEED_OPEN();
  HIPCALL(H.StreamSynchronize(s));
  return AMDC_OK;
}
int amdc_stream_wait_event(void *stream, void *ev) {
  NEED_OPEN();
  HIPCALL(H.StreamWaitEvent(stream, ev, 0));
  return AMDC_OK;
}
int amdc_graph_begin(void *stream) {
  NEED_OPEN();
  if (!stream) return fail(AMDC_EINVAL, "graph_begin: capture needs a created stream, not the default stream");
  HIPCALL(H.StreamBeginCapture(stream, hipStreamCaptureModeRelaxed));
  return AMDC_OK;
}
/* The handle of amdc_graph_end: the executable graph and the graph it was instantiated from. The
 * template stays alive until amdc_graph_destroy: HIP allows destroying it right after
 * instantiation, but a tool that intercepts graph launches (a profiler's launch hook) may look an
 * executable graph's nodes up through it, so nothing a replay can reach is freed before the
 * executable graph itself. */
typedef struct {
  hipGraphExec_t x;
  hipGraph_t g;
} amdc_graph_t;

int amdc_graph_end(void *stream, void **exec) {
  NEED_OPEN();
  if (!exec) return fail(AMDC_EINVAL, "graph_end: exec is NULL");
  *exec = NULL;
  hipGraph_t g = NULL;
  HIPCALL(H.StreamEndCapture(stream, &g));
  amdc_graph_t *h = (amdc_graph_t *)calloc(1, sizeof *h);
  if (!h) {
    H.GraphDestroy(g);
    return fail(AMDC_EHIP, "graph_end: out of host memory");
  }
  const hipError_t e = H.GraphInstantiate(&h->x, g, NULL, NULL, 0);
  if (e) {
    H.GraphDestroy(g);
    free(h);
    return fail(AMDC_EHIP, "hipGraphInstantiate: %s (%d)", H.GetErrorString(e), e);
  }
  h->g = g;
  *exec = h;
  return AMDC_OK;
}
int amdc_graph_launch(void *exec, void *stream) {
  NEED_OPEN();
  if (!exec) return fail(AMDC_EINVAL, "graph_launch: exec is NULL");
  HIPCALL(H.GraphLaunch(((amdc_graph_t *)exec)->x, stream));
  return AMDC_OK;
}
/* Waits for the device first (a replay still queued keeps running on what it holds), then frees
 * the executable graph and its template. */
int amdc_graph_destroy(void *exec) {
  NEED_OPEN();
  if (!exec) return AMDC_OK;
  amdc_graph_t *h = (amdc_graph_t *)exec;
  HIPCALL(H.DeviceSynchronize());
  const hipError_t e1 = H.GraphExecDestroy(h->x), e2 = H.GraphDestroy(h->g);
  free(h);
  if (e1 || e2) return fail(AMDC_EHIP, "graph_destroy: %s", H.GetErrorString(e1 ? e1 : e2));
  return AMDC_OK;
}

/* ---------------------------------------------------------------- launches */

static int g_last_k = -1; /* the kernel of the last launch (amdc_last_kernel) */
static int rec_on(void *stream) { return g_rec.on && stream == g_rec.stream; }
static int rec_put(const amdc_chain_op *o);
static int rec_gemv(int kind, const void *w, const uint8_t *xq, float *y, u32 rows, u32 nb, const float *bias, const float *res) {
  const amdc_chain_op o = {.type = AMDC_CHAIN_GEMV, .kind = kind, .rows = rows, .nb = nb, .w = w, .xq = xq, .y = y, .bias = bias, .res = res};
  return rec_put(&o);
}
static int rec_refuse(int k) {
  g_rec.err = 1;
  return fail(AMDC_EINVAL, "%s cannot be recorded into a chain (amdc_chain_record_begin is on for this stream)", k >= 0 ? kname[k] : "this operator");
}

static int launch_nt(int k, unsigned gx, unsigned gy, unsigned nt, unsigned lds, void *stream, void **args) {
  if (rec_on(stream)) return rec_refuse(k);
  g_last_k = k;
  HIPCALL(H.ModuleLaunchKernel(g_k[k], gx, gy, 1, nt, 1, 1, lds, stream, args, NULL));
  return AMDC_OK;
}
static int launch(int k, unsigned gx, unsigned gy, unsigned lds, void *stream, void **args) { return launch_nt(k, gx, gy, 256u, lds, stream, args); }

const char *amdc_last_kernel(void) { return g_last_k >= 0 ? kname[g_last_k] : ""; }

static int aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

int amdc_quant_q8(const float *x, uint8_t *q, uint32_t nb, uint32_t T, uint32_t xs, uint32_t qs, void *stream) {
  NEED_OPEN();
  if (!x || !q || !nb || !T) return fail(AMDC_EINVAL, "quant_q8: null pointer or empty (nb %u, T %u)", nb, T);
  if (T > 1 && (xs % 4u || qs % 4u || xs < 128u * nb || qs < 40u * nb))
    return fail(AMDC_EINVAL, "quant_q8: strides xs %u, qs %u too small or unaligned for nb %u", xs, qs, nb);
  if (T > 65535u) return fail(AMDC_EINVAL, "quant_q8: T %u > 65535", T);
  if (rec_on(stream) && T == 1u) {
    const amdc_chain_op o = {.type = AMDC_CHAIN_QUANT, .nb = nb, .x = x, .q = q};
    return rec_put(&o);
  }
  void *args[] = {&x, &q, &nb, &xs, &qs};
  return launch(K_QUANT, (nb + 7u) / 8u, T, 0, stream, args);
}

int amdc_rmsnorm_q8(const float *x, const float *w, float *y, uint32_t n, float eps, uint8_t *q, uint32_t T, uint32_t xs, uint32_t ys,
                    uint32_t qs, void *stream) {
  NEED_OPEN();
  if (!x || !w || !y || !n || !T) return fail(AMDC_EINVAL, "rmsnorm_q8: null pointer or empty (n %u, T %u)", n, T);
  if (n % 32u) return fail(AMDC_EINVAL, "rmsnorm_q8: n %u not a multiple of 32", n);
  if (T > 1u && (xs % 4u || ys % 4u || xs < 4u * n || ys < 4u * n || (q && qs < 40u * (n / 32u))))
    return fail(AMDC_EINVAL, "rmsnorm_q8: strides xs %u, ys %u, qs %u too small or unaligned for n %u", xs, ys, qs, n);
  if (T > 65535u) return fail(AMDC_EINVAL, "rmsnorm_q8: T %u > 65535", T);
  if (rec_on(stream) && T == 1u) {
    const amdc_chain_op o = {.type = AMDC_CHAIN_RMSNORM_Q8, .nb = n / 32u, .w = w, .x = x, .q = q, .y = y, .eps = eps};
    return rec_put(&o);
  }
  void *args[] = {&x, &w, &y, &n, &eps, &q, &xs, &ys, &qs};
  return launch(K_RMSNORM_Q8, (n / 32u + 7u) / 8u, T, 0, stream, args);
}

int amdc_swiglu_q8(float *a, const float *b, uint32_t n, uint8_t *q, uint32_t T, uint32_t as, uint32_t qs, void *stream) {
  NEED_OPEN();
  if (!a || !b || !n || !T) return fail(AMDC_EINVAL, "swiglu_q8: null pointer or empty (n %u, T %u)", n, T);
  if (n % 32u) return fail(AMDC_EINVAL, "swiglu_q8: n %u not a multiple of 32", n);
  if (T > 1u && (as % 4u || as < 4u * n || (q && qs < 40u * (n / 32u))))
    return fail(AMDC_EINVAL, "swiglu_q8: strides as %u, qs %u too small or unaligned for n %u", as, qs, n);
  if (T > 65535u) return fail(AMDC_EINVAL, "swiglu_q8: T %u > 65535", T);
  if (rec_on(stream) && T == 1u) {
    const amdc_chain_op o = {.type = AMDC_CHAIN_SWIGLU_Q8, .nb = n / 32u, .x = b, .q = q, .y = a};
    return rec_put(&o);
  }
  void *args[] = {&a, &b, &n, &q, &as, &qs};
  return launch(K_SWIGLU_Q8, (n + 255u) / 256u, T, 0, stream, args);
}

static int check_mat(const char *op, int kind, const void *w, const uint8_t *xq, const float *y, uint32_t rows, uint32_t nb) {
  if (!kind_ok(kind)) return fail(AMDC_EINVAL, "%s: kind %d", op, kind);
  if (!w || !xq || !y) return fail(AMDC_EINVAL, "%s: null pointer", op);
  if (!rows || !nb || rows >= (1u << 24) || nb > 2048u)
    return fail(AMDC_EINVAL, "%s: size %u rows x %u blocks (at most 2^24 - 1 rows and 2048 blocks)", op, rows, nb);
  if ((kind == AMDC_KIND_Q4_K || kind == AMDC_KIND_Q6_K) && nb % 8u)
    return fail(AMDC_EINVAL, "%s: %s needs nb %% 8 == 0 (nb %u)", op, kind == AMDC_KIND_Q4_K ? "Q4_K" : "Q6_K", nb);
  if (!aligned16(w) || !aligned16(xq)) return fail(AMDC_EINVAL, "%s: w and xq must be 16-byte aligned", op);
  return AMDC_OK;
}

/* A lane of the decode kernels holds at most 4 super-groups of its row (its
 * items enter the kernels' ItemTree): L raised until ceil(ng / L) <= 4 (ng <=
 * 256, checked by check_mat). */
static u32 lanes_fit(u32 L, u32 ng) {
  while (L < 64u && (ng + L - 1u) / L > 4u) L <<= 1;
  return L;
}

/* Lanes per row: the smallest power of two >= the super-groups of a row
 * (one super-group per lane), 4..64. */
static u32 gemv_lanes(u32 ng) {
  if (t_lanes > 0) return lanes_fit((u32)t_lanes, ng);
  u32 L = 4;
  while (L < ng && L < 64u) L <<= 1;
  return L;
}

/* Lanes per row of the second decode form: up to 3 super-groups each; for the
 * Q8_0 / Q6_K kinds (k8) then, while the grid has under 2 row groups per CU,
 * more lanes per row and fewer rows per workgroup (measured on MI355X: 1024 x
 * 5120 Q6_K 5.2 us at 32 lanes against 8.6 at 8; 11008 x 4096 Q8_0 11.4 at 16
 * against 12.5 at 8). */
static u32 gemv2_lanes(u32 ng, u32 rows, int k8) {
  const u32 cus = g_cus > 0 ? (u32)g_cus : 256u;
  u32 L = 4u;
  while (L < 64u && 3u * L < ng) L <<= 1;
  while (k8 && L < 64u && L < ng && (rows + 4u * (64u / L) - 1u) / (4u * (64u / L)) < 2u * cus) L <<= 1;
  return t_lanes > 0 ? lanes_fit((u32)t_lanes, ng) : L;
}

/* LDS of the GEMV: 320 bytes per super-group and vector (amdc_kernels.hip). */
#define GEMV_LDS_T1 (150u * 1024u)

static int ws_take(size_t n, void **p);

/* The verify GEMV on int8 MFMA (T <= 16): 64 rows per workgroup, K split
 * over aligned ranges of tiles (64 blocks each): for T <= 8 until the
 * workgroups fill the resident slots about once (Q4 kinds) or the CUs four
 * times (Q8_0, Q6_K), for T > 8 by an estimate of the time. A range holds S
 * tiles, S a power of two <= 4, so that its sum is a subtree of the
 * super-group tree (the kernels' order, equal to the decode GEMV's) and the
 * split sums' tree over the ranges (in the kernel for T <= 8, else
 * amdc_gemm_reduce) completes it. */
static int gemv8_launch(int kind, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                        const float *res, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  const u32 nt = (amdc_ngroups(nb) + 7u) / 8u, wgs = (rows + 63u) / 64u, cus = g_cus > 0 ? (u32)g_cus : 256u;
  /* split K up to one tile of 8 super-groups per workgroup while the grid is under the cap: each
     workgroup's tile is a chain of dependent loads, so more of them in flight win (MI355X, T = 8:
     5120 x 17408 Q4_K 23.6 us at 9 splits against 29.7 at 4, on the 4-wave kernel).
     Q4_0 / Q4_K at T <= 8 (8-wave workgroups, 2 per CU): up to about one round of resident workgroups (10 %
     over: 17408 x 5120 Q4_K T = 8 in 2 splits, 544 workgroups, 20.2 us against 21.1 in 3; the other
     c3 shapes as fast as at their former split) */
  const int q4 = (kind == AMDC_KIND_Q4_0 || kind == AMDC_KIND_Q4_K) && T <= 8u, kv = K_GEMV_Q4K_V8;
  if (q4 && !g_occ[kv] && (H.OccupancyMaxActiveBlocks(&g_occ[kv], g_k[kv], 512, 0) != 0 || g_occ[kv] < 1)) g_occ[kv] = 1;
  const u64 cap = q4 ? (u64)g_occ[kv] * cus * 11u / 10u : 4ull * cus;
  u32 want = 1;
  while (want < nt && (u64)wgs * (want + 1u) <= cap) want++;
  if (t_ksplit > 0) want = (u32)t_ksplit < nt ? (u32)t_ksplit : nt;
  if (want > 16u) want = 16u; /* amdc_gemm_reduce adds at most 16 ranges */
  u32 tps = 1;
  while (tps < 4u && tps * want < nt) tps <<= 1; /* the smallest S with ceil(nt / S) <= want (nt <= 32: S <= 2 for 16) */
  if (T > 8u && t_ksplit <= 0 && wgs < 2u * cus) {
    /* the 16-vector kernels hold one workgroup per CU: the range size S (1, 2, 4 tiles) with the fewest
       tile times, (rounds of workgroups) x S, plus one for the reduction launch of a split; ties to the
       larger S (grids of two workgroups per CU and more are not split). Measured on MI355X (T = 16, us): 11008 x 4096 Q4_0 16.7 unsplit against 20.8 in 2 splits,
       4096 x 11008 Q4_0 19.3 in 3 against 21.4 in 6, 17408 x 5120 Q4_K 33.1 in 3 against 37.8 unsplit */
    u64 best = ~0ull;
    for (u32 S = 4u; S >= 1u; S >>= 1) {
      const u32 n = (nt + S - 1u) / S;
      if (n > 16u) break;
      const u64 est = ((u64)wgs * n + cus - 1u) / cus * (S < nt ? S : nt) + (n > 1u ? 1u : 0u);
      if (est < best) best = est, tps = S;
    }
  }
  /* T <= 8, at most 3 tiles of K, and 3/4 to 1 workgroup per CU: unsplit (no reduction launch), all
     rows in one round. Measured on MI355X (T = 8, us): 16384 x 5120 Q4_K 18.2 unsplit against 20.1
     split 3. (Wider workgroups of 80 or 96 rows, to fit 17408 rows in one round, measured slower:
     24.8 against 21-22 split, their extra waves share the SIMDs.) */
  if (T <= 8u && nt <= 3u && t_ksplit <= 0 && wgs <= cus && 4u * wgs >= 3u * cus) tps = 4u;
  /* T <= 8, 2 tiles of K and at least half a workgroup per CU: unsplit (MI355X, T = 8, us: 11008 x
     4096 Q8_0 14.3 against 15.2-15.4 in 2 splits, Q4_0 12.2 against 12.3) */
  if (T <= 8u && nt == 2u && t_ksplit <= 0 && 2u * wgs >= cus) tps = 2u;
  const u32 ks = (nt + tps - 1u) / tps;
  float *part = NULL;
  if (ks > 1u) {
    int rc = ws_take((size_t)ks * T * rows * 4u, (void **)&part);
    if (rc) return rc;
  }
  /* T <= 8: a split's last workgroup of each row tile adds the partial sums, no reduction launch
     (MI355X, us: 11008 x 4096 Q4_0 12.8 against 13.4, 5120 x 17408 Q4_K 20.7 against 21.0-21.2);
     the 16-vector kernels, one workgroup per CU in several rounds, keep the launch (17408 x 5120
     Q4_K 35.3 against 36.4-36.7 in-kernel: the arrival's round trips delay the next round) */
  u32 *cnt = ks > 1u && T <= 8u && wgs <= AMDC_SPLIT_TILES ? g_split_cnt : NULL;
  void *args[] = {&w, &xq, &y, &rows, &nb, &bias, &res, &T, &xs, &ys, &rs, &part, &tps, &cnt};
  const int v16 = T > 8u; /* the 16-vector form */
  const int k = kind == AMDC_KIND_Q6_K ? (v16 ? K_GEMV_Q6K_V16 : K_GEMV_Q6K_V8)
                : kind == AMDC_KIND_Q4_K ? (v16 ? K_GEMV_Q4K_V16 : K_GEMV_Q4K_V8)
                : kind == AMDC_KIND_Q8_0 ? (v16 ? K_GEMV_Q8_V16 : K_GEMV_Q8_V8)
                                         : (v16 ? K_GEMV_Q4_V16 : K_GEMV_Q4_V8);
  g_last_k = k;
  /* Q4_0 / Q4_K: 8 waves, two per 16 rows, each with half of a tile's super-group pairs */
  const unsigned nth = kind == AMDC_KIND_Q4_0 || kind == AMDC_KIND_Q4_K ? 512u : 256u;
  if (rec_on(stream)) return rec_refuse(k);
  HIPCALL(H.ModuleLaunchKernel(g_k[k], wgs, ks, 1, nth, 1, 1, 0, stream, args, NULL));
  if (ks > 1u && !cnt) {
    const u64 n = (u64)rows * T;
    void *ra[] = {&part, (void *)&ks, &y, &rows, &T, &bias, &res, &ys, &rs};
    return launch(K_GEMM_REDUCE, (unsigned)((n + 255u) / 256u), 1, 0, stream, ra);
  }
  return AMDC_OK;
}

/* The decode GEMV of the Q8_0 and Q6_K kinds (amdc_gemv_q8_0_p2 /
 * amdc_gemv_q6_k_p2: the buffer-load kernel with the lane split of the Q4
 * kinds), one launch per vector: L lanes per row with up to 3 super-groups
 * each, at most 2 workgroups per CU; LDS for the vector (40 or 44 bytes per
 * block) and the workgroup's results. */
static int gemv_k8_launch(int kind, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                          const float *res, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  const u32 ng = amdc_ngroups(nb), bpb = kind == AMDC_KIND_Q6_K ? 44u : 40u;
  const u64 rb = amdc_row_bytes_k(kind, nb);
  if ((u64)rows * rb + rb >= (1ull << 32))
    return fail(AMDC_EINVAL, "gemv: %u rows of %llu bytes: the matrix must be under 4 GiB (split the rows)", rows, (unsigned long long)rb);
  const u32 cus = g_cus > 0 ? (u32)g_cus : 256u, L = gemv2_lanes(ng, rows, 1);
  const u32 rpg = 4u * (64u / L), nrg = (rows + rpg - 1u) / rpg, cap = 2u * cus;
  const unsigned g = t_wgs > 0 && (u32)t_wgs < nrg ? (unsigned)t_wgs : nrg < cap ? nrg : cap;
  const u32 lds = bpb * 8u * ng + 4u * rpg * ((nrg + g - 1u) / g);
  if (lds > GEMV_LDS_T1) return fail(AMDC_EINVAL, "gemv: nb %u too large for the staged vector (%u bytes of LDS)", nb, lds);
  for (u32 t = 0; t < T; t++) {
    const uint8_t *xt = xq + (u64)t * xs;
    float *yt = y + (u64)t * ys;
    const float *rt = res ? res + (u64)t * rs : NULL;
    void *a[] = {&w, &xt, &yt, &rows, &nb, &bias, &rt, (void *)&L};
    int rc = launch(kind == AMDC_KIND_Q6_K ? K_GEMV_Q6K_P2 : K_GEMV_Q8_P2, g, 1, lds, stream, a);
    if (rc) return rc;
  }
  return AMDC_OK;
}

/* Lanes per row of the single-shot decode kernels: the tuning value, else the smallest power of
 * two (4..64) >= the super-groups of a row (one per lane, up to 4 for rows of more than 64).
 * With the quantization in every workgroup (fq), while the grid is over 3 workgroups per CU,
 * half the lanes (two super-groups per lane, half the workgroups: half the quantizations).
 * Measured on MI355X (us, Q8 vector / f32 vector): 22016 x 4096 Q4_0 10.3 / 11.8 (12.5 at 16
 * lanes), 32000 x 4096 13.3 / 15.4; 4096 x 11008 8.1 (64 lanes); 152064 x 5120 Q4_K 72-75. */
static u32 gemvs_lanes(u32 ng, u32 rows, int fq) {
  if (t_lanes > 0) return lanes_fit((u32)t_lanes, ng);
  u32 L = 4u;
  while (L < 64u && L < ng) L <<= 1;
  const u32 cus = g_cus > 0 ? (u32)g_cus : 256u;
  if (fq && L > 4u && (rows + 4u * (64u / L) - 1u) / (4u * (64u / L)) > 3u * cus && (ng + L / 2u - 1u) / (L / 2u) <= 4u) L >>= 1;
  return L;
}

/* The single-shot decode GEMV (amdc_gemv_*_s<NI>; with x: _xs<NI>, the quantization in every
 * workgroup): one row group per workgroup, NI = ceil(ng / L) super-groups per lane, all loaded at
 * once. */
static int gemvs_launch(int kind, const void *w, const void *in, int fq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                        const float *res, uint8_t *q8, void *stream) {
  const u32 ng = amdc_ngroups(nb), L = gemvs_lanes(ng, rows, fq), ni = (ng + L - 1u) / L;
  const u32 rpg = 4u * (64u / L), nrg = (rows + rpg - 1u) / rpg;
  if (ni > 4u) return fail(AMDC_EINVAL, "gemv: %u super-groups on %u lanes (at most 4 per lane)", ng, L);
  const int k = (fq ? K_GEMVXS_Q4 : K_GEMVS_Q4) + (kind == AMDC_KIND_Q4_K ? 4 : 0) + (int)ni - 1;
  if (!fq && ni == 1u && rows >= 16384u) { /* 512-thread workgroups: the vector staged once per 8 waves */
    const u32 rpgw = 8u * (64u / L), nrgw = (rows + rpgw - 1u) / rpgw;
    void *a[] = {&w, &in, &y, &rows, &nb, &bias, &res, (void *)&L};
    return launch_nt(K_GEMVS1W + (kind == AMDC_KIND_Q4_K ? 1 : 0), nrgw, 1, 512u, 320u * ng, stream, a);
  }
  if (fq) {
    void *a[] = {&w, &in, &y, &rows, &nb, &bias, &res, (void *)&L, &q8};
    return launch(k, nrg, 1, 320u * ng, stream, a);
  }
  void *a[] = {&w, &in, &y, &rows, &nb, &bias, &res, (void *)&L};
  return launch(k, nrg, 1, 320u * ng, stream, a);
}

/* The decode GEMV with K split (amdc_gemv_*_k on a Q8 vector, _xk on an f32 one): ranges of R
 * super-groups (a power of two, 4..64), one per workgroup of 4 * 64 / R rows, ceil(ng / R) <= 16
 * ranges; the partial sums in the library's workspace. Returns -1 (nothing launched) where R does
 * not apply. */
static int gemvk_launch(int kind, const void *w, const void *in, int fq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                        const float *res, uint8_t *q8, u32 R, void *stream) {
  const u32 ng = amdc_ngroups(nb), S = (ng + R - 1u) / R, rpg = 4u * (64u / R), nrg = (rows + rpg - 1u) / rpg;
  if (R < 4u || R > 64u || (R & (R - 1u)) || S > 16u || (S > 1u && nrg > AMDC_SPLIT_TILES)) return -1;
  float *part = NULL;
  if (S > 1u) {
    int rc = ws_take((size_t)S * rows * 4u, (void **)&part);
    if (rc) return rc;
  }
  u32 *cnt = g_split_cnt;
  const int k = K_GEMVK_Q4 + (kind == AMDC_KIND_Q4_K ? 2 : 0) + (fq ? 1 : 0);
  if (fq) {
    void *a[] = {&w, &in, &y, &rows, &nb, &bias, &res, (void *)&R, &q8, &part, &cnt};
    return launch(k, nrg, S, 320u * R, stream, a);
  }
  void *a[] = {&w, &in, &y, &rows, &nb, &bias, &res, (void *)&R, &part, &cnt};
  return launch(k, nrg, S, 320u * R, stream, a);
}

static int gemv_launch(int kind, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                       const float *res, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  if (kind == AMDC_KIND_Q8_0 || kind == AMDC_KIND_Q6_K) {
    if (T == 1u || t_unroll > 0) return gemv_k8_launch(kind, w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
    if (T <= 8u && t_ksplit == 0) {
      /* a few vectors on a small matrix: the decode items and arithmetic for every vector
         (amdc_gemv_{q8_0,q6_k}_m1), one launch, the vectors in LDS, one super-group per lane (the
         kernels with two hold 229 / 321 VGPRs) */
      const u32 ng = amdc_ngroups(nb), bpb = kind == AMDC_KIND_Q6_K ? 44u : 40u, lds = bpb * 8u * ng * T;
      u32 L = 4u;
      while (L < 64u && L < ng) L <<= 1;
      const u32 ni = (ng + L - 1u) / L, rpg = 4u * (64u / L), nrg = (rows + rpg - 1u) / rpg;
      const u64 rb = amdc_row_bytes_k(kind, nb);
      /* measured on MI355X (us, this kernel / the MFMA verify kernel): Q6_K 1024 x 5120 T = 2, 4, 8 5.2 /
         14.3, 6.9 / 14.4, 10.3 / 17.8; 4096 x 4096 6.6 / 15.4, 8.2 / 15.4, 11.5 / 18.6; 6144 x 5120 T = 4
         15.7 / 17.2. Q8_0 4096 x 4096 6.4 / 9.5, 7.8 / 9.6, 10.6 / 10.1; 11008 x 4096 T = 2, 4 12.3 /
         15.2, 15.4 / 14.9; 1024 x 2048 T = 8 7.6 / 6.5: Q8_0 only up to T = 4 and half the size */
      const u64 lim = kind == AMDC_KIND_Q6_K ? M8_MAX : T <= 4u ? M8_MAX * 2u / 3u : 0u;
      if (ni == 1u && lds <= 64u * 1024u && (u64)T * rows * ng <= lim && (u64)rows * rb + rb < (1ull << 32)) {
        void *a[] = {&w, &xq, &y, &rows, &nb, &bias, &res, (void *)&L, &T, &xs, &ys, &rs};
        return launch(K_GEMVM8 + (kind == AMDC_KIND_Q6_K ? 1 : 0), nrg, 1, lds, stream, a);
      }
    }
  } else if (T > 1u && t_unroll > 0) { /* tuning: one decode launch per vector */
    for (u32 t = 0; t < T; t++) {
      int rc = gemv_launch(kind, w, xq + (u64)t * xs, y + (u64)t * ys, rows, nb, bias, res ? res + (u64)t * rs : NULL, 1u, 0u, 0u, 0u, stream);
      if (rc) return rc;
    }
    return AMDC_OK;
  }
  if (T > 1u && T <= 8u && (kind == AMDC_KIND_Q4_0 || kind == AMDC_KIND_Q4_K) && t_ksplit == 0) {
    /* a few vectors on a small matrix: the decode kernel's dots for every vector (amdc_gemv_*_m1), one
       launch, no K split; the int8-MFMA kernels below cost about 11 us at any size (the K split and the
       reduction launch). Measured on MI355X (us, this kernel / the MFMA kernels): T = 2 17408 x 5120
       Q4_K 20.7 / 21.3, 11008 x 4096 Q4_0 9.8 / 13.2; T = 4 6144 x 5120 Q4_K 11.7 / 12.2, 11008 x 4096
       12.6 / 13.0, 17408 x 5120 26.0 / 21.5; T = 8 4096 x 4096 Q4_0 10.1 / 11.4, 6144 x 5120 Q4_K
       17.4 / 12.3. One super-group per lane (up to 64 per row), LDS for every vector. */
    const u32 ng = amdc_ngroups(nb), L = gemvs_lanes(ng, rows, 0), rpg = 4u * (64u / L), lds = 320u * ng * T;
    if (ng <= L && (u64)T * rows * ng <= 786432u && lds <= 64u * 1024u) {
      const u32 nrg = (rows + rpg - 1u) / rpg;
      void *a[] = {&w, &xq, &y, &rows, &nb, &bias, &res, (void *)&L, &T, &xs, &ys, &rs};
      return launch(K_GEMVM_Q4 + (kind == AMDC_KIND_Q4_K ? 1 : 0), nrg, 1, lds, stream, a);
    }
  }
  if (T > 1u) {
    /* the int8-MFMA verify kernels, up to 16 vectors per launch; measured on MI355X, T = 16:
       17408 x 5120 Q4_K 30.8 us in one launch, 41 us as two 8-vector launches, 176 us on the dot4
       multi-vector kernel */
    for (u32 t0 = 0; t0 < T; t0 += 16u) {
      const u32 tn = T - t0 < 16u ? T - t0 : 16u;
      int rc = gemv8_launch(kind, w, xq + (u64)t0 * xs, y + (u64)t0 * ys, rows, nb, bias, res ? res + (u64)t0 * rs : NULL, tn, xs, ys, rs,
                            stream);
      if (rc) return rc;
    }
    return AMDC_OK;
  }
  const u32 ng = amdc_ngroups(nb), L = gemv_lanes(ng), rpg = 4u * (64u / L), nrg = (rows + rpg - 1u) / rpg;
  if (t_form == 4) { /* tuning: the K-split form, ranges of t_lanes super-groups */
    const int rc = gemvk_launch(kind, w, xq, 0, y, rows, nb, bias, res, NULL, t_lanes > 0 ? (u32)t_lanes : 8u, stream);
    if (rc != -1) return rc;
  }
  /* the single-shot kernels (form 3) by default: up to 256 super-groups per row */
  const int form = t_form > 0 && t_form != 4 ? t_form : ng <= 256u ? 3 : 2;
  if (form == 3) return gemvs_launch(kind, w, xq, 0, y, rows, nb, bias, res, NULL, stream);
  if (form == 2 && (u64)rows * 144u * ng + 144u * ng < (1ull << 32)) {
    /* the decode kernel with buffer loads (32-bit offsets: matrices under 4 GiB), for long rows: up
       to 3 super-groups per lane (it keeps the next one in flight), at most 2 workgroups per CU; LDS
       for the vector and the workgroup's results. Measured on MI355X: 4096 x 11008 Q4_0 8.6 us (9.5 with the
       amdc_gemv_*_p1 split), 5120 x 17408 Q4_K 14.7 (15.8). */
    const u32 L2 = gemv2_lanes(ng, rows, 0);
    const u32 rpg2 = 4u * (64u / L2), nrg2 = (rows + rpg2 - 1u) / rpg2, cap = 2u * (g_cus > 0 ? (u32)g_cus : 256u);
    const unsigned g2 = t_wgs > 0 && (u32)t_wgs < nrg2 ? (unsigned)t_wgs : nrg2 < cap ? nrg2 : cap;
    const u32 lds2 = 320u * ng + 4u * rpg2 * ((nrg2 + g2 - 1u) / g2);
    if (lds2 > GEMV_LDS_T1) return fail(AMDC_EINVAL, "gemv: %u rows x %u blocks: %u bytes of LDS (more workgroups)", rows, nb, lds2);
    void *a2[] = {&w, &xq, &y, &rows, &nb, &bias, &res, (void *)&L2};
    return launch(kind == AMDC_KIND_Q4_K ? K_GEMV_Q4K_P2 : K_GEMV_Q4_P2, g2, 1, lds2, stream, a2);
  }
  /* the pipelined decode kernel (320 ng bytes of LDS: ng <= 256 fits) */
  const unsigned g1 = t_wgs > 0 && (u32)t_wgs < nrg ? (unsigned)t_wgs : nrg;
  void *a1[] = {&w, &xq, &y, &rows, &nb, &bias, &res, (void *)&L};
  return launch(kind == AMDC_KIND_Q4_K ? K_GEMV_Q4K_P1 : K_GEMV_Q4_P1, g1, 1, 320u * ng, stream, a1);
}

int amdc_gemv_q4(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                 void *stream) {
  NEED_OPEN();
  int rc = check_mat("gemv_q4", AMDC_KIND_Q4_0, w, xq, y, rows, nb);
  if (!rc && rec_on(stream)) return rec_gemv(AMDC_KIND_Q4_0, w, xq, y, rows, nb, bias, res);
  return rc ? rc : gemv_launch(AMDC_KIND_Q4_0, w, xq, y, rows, nb, bias, res, 1, 0, 0, 0, stream);
}

int amdc_gemv_q4k(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                  void *stream) {
  NEED_OPEN();
  int rc = check_mat("gemv_q4k", AMDC_KIND_Q4_K, w, xq, y, rows, nb);
  if (!rc && rec_on(stream)) return rec_gemv(AMDC_KIND_Q4_K, w, xq, y, rows, nb, bias, res);
  return rc ? rc : gemv_launch(AMDC_KIND_Q4_K, w, xq, y, rows, nb, bias, res, 1, 0, 0, 0, stream);
}

static int check_t(const char *op, uint32_t nb, uint32_t rows, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, const float *res) {
  if (!T) return fail(AMDC_EINVAL, "%s: T == 0", op);
  if (T > 1u && (xs % 16u || xs < 40u * nb)) return fail(AMDC_EINVAL, "%s: xs %u (a multiple of 16, >= 40 nb = %u)", op, xs, 40u * nb);
  if (T > 1u && ys < rows) return fail(AMDC_EINVAL, "%s: ys %u < rows %u", op, ys, rows);
  if (T > 1u && res && rs < rows) return fail(AMDC_EINVAL, "%s: rs %u < rows %u", op, rs, rows);
  return AMDC_OK;
}

static int gemv_t(int kind, const char *op, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                  const float *res, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  NEED_OPEN();
  int rc = check_mat(op, kind, w, xq, y, rows, nb);
  if (!rc) rc = check_t(op, nb, rows, T, xs, ys, rs, res);
  for (u32 t0 = 0; !rc && t0 < T; t0 += 16u) { /* 16 vectors per gemv_launch (the dot4 kernels' most; the MFMA kernels take 8) */
    const u32 tn = T - t0 < 16u ? T - t0 : 16u;
    rc = gemv_launch(kind, w, xq + (u64)t0 * xs, y + (u64)t0 * ys, rows, nb, bias, res ? res + (u64)t0 * rs : NULL, tn, xs, ys, rs,
                     stream);
  }
  return rc;
}

/* The decode GEMV of an f32 input: where one workgroup can hold a CU's share
 * of the rows (gemvxw_pick), one launch of about one workgroup per CU that
 * quantizes the vector once per CU in its prologue; else, for nb <= x_fuse_nb
 * (128 by default), one launch whose 256-thread workgroups quantize the
 * vector in their prologue (the quantization then hides under the weight
 * loads); for larger nb, where that prologue costs more than a launch,
 * amdc_quant_q8 into q8 (or the library's workspace when q8 is NULL) and the
 * GEMV. Measured on MI355X (single-shot kernels): 4096 x 4096 Q4_0 4.5 us
 * fused against 6.0 us for the two launches, 12288 x 4096 7.9 against 8.8,
 * 22016 x 4096 11.8 against 12.2. */
/* The workgroup-per-CU form of the fused quantization (amdc_gemv_q4_0_xw1, amdc_gemv_q4_k_xw1 /
 * _xw2): the lanes per row L, super-groups per lane ni and threads nth such that one workgroup
 * holds the rows of one CU's share, for more than 4 and at most 16 waves (Q4_0: one super-group
 * per lane only); 0 when no such size exists (the 256-thread kernels then). Measured on MI355X, f32
 * input, Q4_0 (us, this form / the 256-thread kernels): 12288 x 4096 7.6 / 8.4, 4096 x 11008 9.3 /
 * 10.7 (there against a separate quantization launch); 22016 x 4096 on two super-groups per lane
 * 12.7 / 12.3 (not taken). */
static int gemvxw_pick(int kind, u32 ng, u32 rows, u32 *L, u32 *ni, u32 *nth) {
  const u32 cus = g_cus > 0 ? (u32)g_cus : 256u, rpc = (rows + cus - 1u) / cus;
  for (u32 n = 1u; n <= (kind == AMDC_KIND_Q4_0 ? 1u : 2u); n++) {
    u32 l = 4u;
    while (l < 64u && l * n < ng) l <<= 1;
    if ((ng + l - 1u) / l != n) continue;
    const u32 rpw = 64u / l, waves = (rpc + rpw - 1u) / rpw;
    if (waves > 4u && waves <= 16u) {
      *L = l, *ni = n, *nth = 64u * waves;
      return 1;
    }
  }
  return 0;
}

static int gemv_x(int kind, const char *op, const void *w, const float *x, float *y, uint32_t rows, uint32_t nb, const float *bias,
                  const float *res, uint8_t *q8, void *stream) {
  NEED_OPEN();
  int rc = check_mat(op, kind, w, (const uint8_t *)x, y, rows, nb);
  if (rc) return rc;
  if (q8 && !aligned16(q8)) return fail(AMDC_EINVAL, "%s: q8 must be 16-byte aligned", op);
  if (rec_on(stream)) {
    /* with q8: the quantization into q8 (which the caller may read) and the GEMV on it; without: one
       operation that quantizes in every workgroup (Q4_0 / Q4_K) */
    if (q8) {
      const amdc_chain_op o = {.type = AMDC_CHAIN_QUANT, .nb = nb, .x = x, .q = q8};
      return (rc = rec_put(&o)) ? rc : rec_gemv(kind, w, q8, y, rows, nb, bias, res);
    }
    if (kind != AMDC_KIND_Q4_0 && kind != AMDC_KIND_Q4_K) {
      g_rec.err = 1;
      return fail(AMDC_EINVAL, "%s: pass q8 to record a Q8_0 / Q6_K GEMV of an f32 vector", op);
    }
    const amdc_chain_op o = {.type = AMDC_CHAIN_GEMV_X, .kind = kind, .rows = rows, .nb = nb, .w = w, .x = x, .y = y, .bias = bias, .res = res};
    return rec_put(&o);
  }
  const u32 ng = amdc_ngroups(nb), L = gemv_lanes(ng), rpg = 4u * (64u / L), nrg = (rows + rpg - 1u) / rpg;
  if ((kind == AMDC_KIND_Q4_0 || kind == AMDC_KIND_Q4_K) && t_form == 4) { /* tuning: the K-split form */
    rc = gemvk_launch(kind, w, x, 1, y, rows, nb, bias, res, q8, t_lanes > 0 ? (u32)t_lanes : 8u, stream);
    if (rc != -1) return rc;
  }
  u32 Lw, niw, nthw;
  if ((kind == AMDC_KIND_Q4_0 || kind == AMDC_KIND_Q4_K) && (t_form == 0 || t_form == 3) && t_lanes <= 0 && t_wgs <= 0 &&
      320u * ng <= GEMV_LDS_T1 && gemvxw_pick(kind, ng, rows, &Lw, &niw, &nthw)) {
    const u32 rpgw = (nthw / 64u) * (64u / Lw), gw = (rows + rpgw - 1u) / rpgw;
    void *a[] = {&w, &x, &y, &rows, &nb, &bias, &res, (void *)&Lw, &q8};
    return launch_nt(kind == AMDC_KIND_Q4_K ? K_GEMVXW_Q4 + (int)niw : K_GEMVXW_Q4, gw, 1, nthw, 320u * ng, stream, a);
  }
  if (kind == AMDC_KIND_Q4_K && nb > x_fuse_nb && rows <= 8192u && t_form == 0 && t_lanes <= 0 && t_wgs <= 0) {
    /* long Q4_K rows on few rows: the K-split form, 8 super-groups per range, quantizing its slice in
       every workgroup, instead of a quantize launch and the GEMV. Measured on MI355X (us, f32 input,
       K-split at 4 / 8 / 16 / 32 super-groups per range against the two launches): 5120 x 17408 -- /
       14.1 / 16.3 / 22.9 against 16.6; 34816 x 5120 27.6 (8) against 21.9, 6144 x 5120 and the Q4_0
       shapes slower than their fused kernels, so only here. */
    rc = gemvk_launch(kind, w, x, 1, y, rows, nb, bias, res, q8, 8u, stream);
    if (rc != -1) return rc;
  }
  if (nb > x_fuse_nb || 320u * ng > GEMV_LDS_T1 || kind == AMDC_KIND_Q8_0 || kind == AMDC_KIND_Q6_K) {
    if (!q8) {
      if ((rc = ws_take((size_t)40u * nb + 64u, (void **)&q8))) return rc;
    }
    if ((rc = amdc_quant_q8(x, q8, nb, 1u, 0u, 0u, stream))) return rc;
    return gemv_t(kind, op, w, q8, y, rows, nb, bias, res, 1u, 0u, 0u, 0u, stream);
  }
  if (t_form == 0 || t_form == 3) return gemvs_launch(kind, w, x, 1, y, rows, nb, bias, res, q8, stream);
  /* every workgroup quantizes the whole vector first: a persistent grid of at most 3 workgroups
     per CU (each loops over row groups) pays that once per slot */
  const u32 cap = 3u * (g_cus > 0 ? (u32)g_cus : 256u);
  const unsigned grid = t_wgs > 0 && (u32)t_wgs < nrg ? (unsigned)t_wgs : nrg < cap ? nrg : cap;
  void *args[] = {&w, &x, &y, &rows, &nb, &bias, &res, (void *)&L, &q8};
  return launch(kind == AMDC_KIND_Q4_K ? K_GEMV_Q4K_X1 : K_GEMV_Q4_X1, grid, 1, 320u * ng, stream, args);
}

int amdc_gemv_q4_x(const void *w, const float *x, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res, uint8_t *q8,
                   void *stream) {
  return gemv_x(AMDC_KIND_Q4_0, "gemv_q4_x", w, x, y, rows, nb, bias, res, q8, stream);
}

int amdc_gemv_q4k_x(const void *w, const float *x, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res, uint8_t *q8,
                    void *stream) {
  return gemv_x(AMDC_KIND_Q4_K, "gemv_q4k_x", w, x, y, rows, nb, bias, res, q8, stream);
}

int amdc_gemv_q4_t(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                   uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  return gemv_t(AMDC_KIND_Q4_0, "gemv_q4_t", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
}

int amdc_gemv_q4k_t(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                    uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  return gemv_t(AMDC_KIND_Q4_K, "gemv_q4k_t", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
}

int amdc_gemv_q8(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                 void *stream) {
  NEED_OPEN();
  int rc = check_mat("gemv_q8", AMDC_KIND_Q8_0, w, xq, y, rows, nb);
  if (!rc && rec_on(stream)) return rec_gemv(AMDC_KIND_Q8_0, w, xq, y, rows, nb, bias, res);
  return rc ? rc : gemv_launch(AMDC_KIND_Q8_0, w, xq, y, rows, nb, bias, res, 1, 0, 0, 0, stream);
}

int amdc_gemv_q6k(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                  void *stream) {
  NEED_OPEN();
  int rc = check_mat("gemv_q6k", AMDC_KIND_Q6_K, w, xq, y, rows, nb);
  if (!rc && rec_on(stream)) return rec_gemv(AMDC_KIND_Q6_K, w, xq, y, rows, nb, bias, res);
  return rc ? rc : gemv_launch(AMDC_KIND_Q6_K, w, xq, y, rows, nb, bias, res, 1, 0, 0, 0, stream);
}

/* The decode GEMV with the fused RMSNorm tail: the single-shot kernels (Q4_0 / Q4_K) or the second
 * form (Q8_0, Q6_K), with the lane split of amdc_gemv_* (the same y), whose last workgroup writes ny
 * and nq as amdc_rmsnorm_q8 of y. */
int amdc_gemv_norm(int kind, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                   const float *nw, float *ny, uint8_t *nq, float eps, void *stream) {
  NEED_OPEN();
  int rc = check_mat("gemv_norm", kind, w, xq, y, rows, nb);
  if (rc) return rc;
  if (!nw || !ny) return fail(AMDC_EINVAL, "gemv_norm: nw and ny are required");
  if (rows % 32u || rows > 8192u) return fail(AMDC_EINVAL, "gemv_norm: rows %u (a multiple of 32, the norm's Q8 blocks, at most 8192)", rows);
  if (!(eps >= 0.0f)) return fail(AMDC_EINVAL, "gemv_norm: eps must be >= 0");
  const u32 ng = amdc_ngroups(nb);
  if (kind == AMDC_KIND_Q4_0 || kind == AMDC_KIND_Q4_K) { /* check_mat: nb <= 2048, so ng <= 256 */
    const u32 L = gemvs_lanes(ng, rows, 0), ni = (ng + L - 1u) / L, rpg = 4u * (64u / L), nrg = (rows + rpg - 1u) / rpg;
    if (ni > 4u) return fail(AMDC_EINVAL, "gemv_norm: %u super-groups on %u lanes (at most 4 per lane)", ng, L);
    void *a[] = {&w, &xq, &y, &rows, &nb, &bias, &res, (void *)&L, &nw, &ny, &nq, &eps, &g_norm_cnt};
    return launch(K_GEMVSN_Q4 + (kind == AMDC_KIND_Q4_K ? 4 : 0) + (int)ni - 1, nrg, 1, 320u * ng, stream, a);
  }
  const u64 rb = amdc_row_bytes_k(kind, nb);
  if ((u64)rows * rb + rb >= (1ull << 32))
    return fail(AMDC_EINVAL, "gemv_norm: %u rows of %llu bytes: the matrix must be under 4 GiB", rows, (unsigned long long)rb);
  /* the lane split of the T = 1 launch of gemv_k8_launch */
  const u32 L = gemv2_lanes(ng, rows, 1), rpg = 4u * (64u / L), nrg = (rows + rpg - 1u) / rpg;
  const u32 cap = 2u * (g_cus > 0 ? (u32)g_cus : 256u), g = nrg < cap ? nrg : cap;
  const u32 lds = (kind == AMDC_KIND_Q6_K ? 352u : 320u) * ng + 4u * rpg * ((nrg + g - 1u) / g);
  if (lds > GEMV_LDS_T1) return fail(AMDC_EINVAL, "gemv_norm: nb %u too large for the staged vector (%u bytes of LDS)", nb, lds);
  const int k = K_GEMV2N + (kind == AMDC_KIND_Q6_K ? 1 : 0);
  void *a[] = {&w, &xq, &y, &rows, &nb, &bias, &res, (void *)&L, &nw, &ny, &nq, &eps, &g_norm_cnt};
  return launch(k, g, 1, lds, stream, a);
}

int amdc_gemv_q8_t(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                   uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  return gemv_t(AMDC_KIND_Q8_0, "gemv_q8_t", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
}

int amdc_gemv_q6k_t(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                    uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  return gemv_t(AMDC_KIND_Q6_K, "gemv_q6k_t", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
}

int amdc_gemv_q8_x(const void *w, const float *x, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res, uint8_t *q8,
                   void *stream) {
  return gemv_x(AMDC_KIND_Q8_0, "gemv_q8_x", w, x, y, rows, nb, bias, res, q8, stream);
}

int amdc_gemv_q6k_x(const void *w, const float *x, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res, uint8_t *q8,
                    void *stream) {
  return gemv_x(AMDC_KIND_Q6_K, "gemv_q6k_x", w, x, y, rows, nb, bias, res, q8, stream);
}

/* Grow the workspace to at least n bytes (a power of two, >= 1 MiB). A smaller
 * workspace is kept, not freed, until amdc_close: a graph captured earlier may
 * still hold its address, and replays of it must stay valid. */
static int ws_reserve(size_t n) {
  if (n <= g_ws_bytes) return AMDC_OK;
  size_t m = (size_t)1 << 20;
  while (m < n) m <<= 1;
  if (g_ws) {
    if (g_ws_old_n == sizeof g_ws_old / sizeof g_ws_old[0]) return fail(AMDC_EINVAL, "workspace: grown too many times");
    g_ws_old[g_ws_old_n++] = g_ws;
  }
  g_ws = NULL, g_ws_bytes = 0;
  HIPCALL(H.Malloc(&g_ws, m));
  g_ws_bytes = m;
  return AMDC_OK;
}

/* The workspace of an operator: n bytes at *p, from the grown allocation, or from the fixed
 * scratch array inside amdc_op_gemv_noalloc. Every caller asks before its first launch, so a
 * rejected request launches nothing. No operator needs its workspace to start at zero. */
static int ws_take(size_t n, void **p) {
  if (g_ws_fixed) {
    if (n > g_scratch_bytes)
      return fail(AMDC_EINVAL, "op_gemv_noalloc: needs %zu bytes of workspace, the scratch array holds %zu (%u MiB)", n, g_scratch_bytes,
                  (unsigned)(AMDC_SCRATCH_BYTES >> 20));
    *p = g_scratch;
    return AMDC_OK;
  }
  int rc = ws_reserve(n);
  if (!rc) *p = g_ws;
  return rc;
}

/* The f16-MFMA GEMM kernels: rows x tokens per workgroup. */
static const struct {
  int k;
  u32 mr, nt, threads;
} gh[3] = {{K_GEMMH_M64_N128, 64, 128, 256}, {K_GEMMH_M64_N64, 64, 64, 256}, {K_GEMMH_M128, 128, 128, 512}};

/* The prefill GEMM on the f16-MFMA kernels (every kind). */
static int gemm_launch(int kind, const char *op, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                       const float *res, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  NEED_OPEN();
  int rc = check_mat(op, kind, w, xq, y, rows, nb);
  if (!rc) rc = check_t(op, nb, rows, T, xs, ys, rs, res);
  if (rc) return rc;
  if (T == 1u) xs = 40u * nb, ys = rows, rs = rows; /* one row: the strides are not used */
  if (xs % 16u) return fail(AMDC_EINVAL, "%s: xs %u not a multiple of 16", op, xs);
  if (kind == AMDC_KIND_Q4_K && (t_gemm == 1 || t_gemm == 2)) { /* the int8-MFMA kernel */
    const u32 n = t_gemm == 2 ? 128u : 64u;
    const u64 grid = (u64)((rows + 63u) / 64u) * ((T + n - 1u) / n);
    if (grid > 0x7FFFFFFFull) return fail(AMDC_EINVAL, "gemm_q4k: grid too large");
    void *args[] = {&w, &xq, &y, &rows, &nb, &bias, &res, &T, &xs, &ys, &rs};
    return launch(n == 128u ? K_GEMM_N128 : K_GEMM_N64, (unsigned)grid, 1, 0, stream, args);
  }
  /* the f16-MFMA kernel: 128 tokens per workgroup when there are that many */
  const u32 ng = amdc_ngroups(nb), cus = g_cus > 0 ? (u32)g_cus : 256u;
  /* 64-token tiles for Q4_0 at any T (its 128-token kernel holds 284 VGPRs, one wave per SIMD:
     measured 150 / 188 TOPS against 140 / 169 on 11008 x 4096 / 4096 x 11008, T = 256) */
  /* Q4_K with more than 64 tokens: 128-row tiles below 65536 rows (amdc_gemmh_m128_n128 lists the
     measurements) */
  int v = t_gemm >= 3 ? t_gemm - 3 : (T > 64u && kind != AMDC_KIND_Q4_0 ? (kind == AMDC_KIND_Q4_K && rows < 65536u ? 2 : 0) : 1);
  if (v >= 2 && kind != AMDC_KIND_Q4_K) v = 0; /* the 128-row tile is built for Q4_K */
  const int kk = kind == AMDC_KIND_Q8_0 ? (v ? K_GEMMH_Q8_N64 : K_GEMMH_Q8_N128)
                 : kind == AMDC_KIND_Q6_K ? (v ? K_GEMMH_Q6K_N64 : K_GEMMH_Q6K_N128)
                 : kind == AMDC_KIND_Q4_0 ? (v ? K_GEMMH_Q4_N64 : K_GEMMH_Q4_N128)
                                          : gh[v].k;
  const u32 ntt = (T + gh[v].nt - 1u) / gh[v].nt, tiles = (rows + gh[v].mr - 1u) / gh[v].mr * ntt;
  /* the schedule: whole rounds of resident workgroups (occupancy x CUs) run
   * their tiles over the whole K; the tiles left over (whole row tiles) are
   * split in K to fill part of one more round (a 544-tile matrix on 512
   * slots ran at 221-242 TOPS, a 512-tile one at 323). A tuning K split
   * splits every tile instead. */
  u32 nfull, ks;
  if (t_ksplit > 0) {
    nfull = 0, ks = (u32)t_ksplit;
  } else {
    if (!g_occ[kk] && (H.OccupancyMaxActiveBlocks(&g_occ[kk], g_k[kk], (int)gh[v].threads, 0) != 0 || g_occ[kk] < 1))
      g_occ[kk] = 1;
    const u64 cap = (u64)g_occ[kk] * cus;
    nfull = (u32)((u64)tiles / cap * cap / ntt * ntt);
    const u32 tail = tiles - nfull;
    /* after whole rounds the tail fills half a round (MI355X, 17408 x 5120 T = 256: a tail of 32
       tiles in 8 splits 302 TOPS, in 16 292); alone, a whole round */
    ks = tail ? (u32)(cap / ((nfull ? 2u : 1u) * tail)) : 1u;
    if (ks < 1u) ks = 1u;
  }
  if (ks > ng) ks = ng;
  if (ks > 16u) ks = 16u; /* amdc_gemm_reduce adds at most 16 splits */
  if (ks == 1u) nfull = tiles;
  const u32 r0 = nfull / ntt * gh[v].mr, trows = rows - r0; /* the split tail's rows */
  const u32 Tp = (T + 127u) / 128u * 128u, K = 32u * nb;
  const size_t xh_b = (size_t)Tp * K * 2u, sc_b = (size_t)nb * Tp * 4u, part_b = ks > 1u ? (size_t)ks * T * trows * 4u : 0u;
  uint8_t *ws = NULL;
  rc = ws_take(xh_b + 2u * sc_b + part_b, (void **)&ws);
  if (rc) return rc;
  void *xh = ws, *da = ws + xh_b, *xa = ws + xh_b + sc_b, *part = ks > 1u ? (void *)(ws + xh_b + 2u * sc_b) : NULL;
  void *pa[] = {&xq, &nb, &T, &xs, &xh, &da, &xa, (void *)&Tp};
  rc = launch(K_Q8_PREP, (unsigned)((nb + 7u) / 8u * (Tp / 32u)), 1, 0, stream, pa); /* 8 blocks x 32 tokens per workgroup */
  if (rc) return rc;
  const u64 grid = (u64)nfull + (u64)(tiles - nfull) * ks;
  if (grid > 0x7FFFFFFFull) return fail(AMDC_EINVAL, "%s: grid too large", op);
  void *ga[] = {&w, &xh, &da, &xa, &y, &rows, &nb, &bias, &res, &T, (void *)&Tp, &ys, &rs, &part, &nfull, &ks};
  g_last_k = kk;
  if (rec_on(stream)) return rec_refuse(kk);
  HIPCALL(H.ModuleLaunchKernel(g_k[kk], (unsigned)grid, 1, 1, gh[v].threads, 1, 1, 0, stream, ga, NULL));
  if (ks > 1u) { /* the tail rows: y, bias and res from row r0 */
    const u64 n = (u64)trows * T;
    float *yt = y + r0;
    const float *bt = bias ? bias + r0 : NULL, *rt = res ? res + r0 : NULL;
    void *ra[] = {&part, &ks, &yt, (void *)&trows, &T, &bt, &rt, &ys, &rs};
    return launch(K_GEMM_REDUCE, (unsigned)((n + 255u) / 256u), 1, 0, stream, ra);
  }
  return AMDC_OK;
}

int amdc_gemm_q4k(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                  uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  return gemm_launch(AMDC_KIND_Q4_K, "gemm_q4k", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
}

int amdc_gemm_q4(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                 uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  return gemm_launch(AMDC_KIND_Q4_0, "gemm_q4", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
}

int amdc_gemm_q8(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                 uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  return gemm_launch(AMDC_KIND_Q8_0, "gemm_q8", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
}

int amdc_gemm_q6k(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                  uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  return gemm_launch(AMDC_KIND_Q6_K, "gemm_q6k", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
}

/* op_gemv's choice for T > 1: the prefill GEMM or the verify kernels (up to 16 vectors per
 * launch). IE_GEMM_MIN set (> 0): the reference's rule, T >= IE_GEMM_MIN. Else measured on
 * MI355X (us per call, verify / GEMM): the verify kernels win up to T = 32 on the 7B-27B layer
 * shapes (17408 x 5120 Q4_K T = 32: 60 / 70, T = 33: 70 / 70, T = 40: 79 / 71; 4096 x 11008
 * Q4_0 T = 32: 36 / 43; 5120 x 6144 Q4_K T = 32: 32 / 37), except on matrices of at most 2^24
 * weights, where the GEMM wins from T = 20 (4096 x 4096 Q4_0 T = 20: 27 / 23, T = 17: 19 / 22;
 * Q8_0 T = 20: 29 / 27). */
static int use_gemm(uint32_t T, uint32_t rows, uint32_t nb) {
  if (t_gemm_min > 0) return (int)T >= t_gemm_min;
  if (T >= 33u) return 1;
  return T >= 20u && (u64)rows * nb * 32u <= (1ull << 24);
}

int amdc_op_gemv(int kind, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                 const float *res, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  NEED_OPEN();
  if (T == 1u) {
    int rc = check_mat("op_gemv", kind, w, xq, y, rows, nb);
    if (!rc && rec_on(stream)) return rec_gemv(kind, w, xq, y, rows, nb, bias, res);
    return rc ? rc : gemv_launch(kind, w, xq, y, rows, nb, bias, res, 1, 0, 0, 0, stream);
  }
  if (use_gemm(T, rows, nb)) return gemm_launch(kind, "op_gemv", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
  return gemv_t(kind, "op_gemv", w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
}

int amdc_op_gemv_noalloc(int kind, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                         const float *res, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream) {
  NEED_OPEN();
  g_ws_fixed = 1;
  const int rc = amdc_op_gemv(kind, w, xq, y, rows, nb, bias, res, T, xs, ys, rs, stream);
  g_ws_fixed = 0;
  return rc;
}

int amdc_block_dots(int kind, const void *w, const uint8_t *xq, int32_t *out, uint32_t rows, uint32_t nb, void *stream) {
  NEED_OPEN();
  int rc = check_mat("block_dots", kind, w, xq, (const float *)out, rows, nb);
  if (rc) return rc;
  const u64 n = (u64)rows * nb;
  if ((n + 255u) / 256u > 0x7FFFFFFFull) return fail(AMDC_EINVAL, "block_dots: too large");
  void *args[] = {&w, &xq, &out, &rows, &nb};
  const int k = kind == AMDC_KIND_Q4_K ? K_DOTS_Q4K : kind == AMDC_KIND_Q8_0 ? K_DOTS_Q8 : kind == AMDC_KIND_Q6_K ? K_DOTS_Q6K : K_DOTS_Q4;
  return launch(k, (unsigned)((n + 255u) / 256u), 1, 0, stream, args);
}

int amdc_probe_read(const void *src, size_t nbytes, void *scratch, uint32_t grid, void *stream) {
  NEED_OPEN();
  if (!src || !scratch || nbytes % 16u || !aligned16(src) || !grid) return fail(AMDC_EINVAL, "probe_read: bad arguments");
  u64 n = nbytes / 16u;
  void *args[] = {&src, &n, &scratch};
  return launch(K_PROBE_READ, grid, 1, 0, stream, args);
}

int amdc_probe_copy(void *dst, const void *src, size_t nbytes, uint32_t grid, void *stream) {
  NEED_OPEN();
  if (!src || !dst || nbytes % 16u || !aligned16(src) || !aligned16(dst) || !grid) return fail(AMDC_EINVAL, "probe_copy: bad arguments");
  u64 n = nbytes / 16u;
  void *args[] = {&src, &dst, &n};
  return launch(K_PROBE_COPY, grid, 1, 0, stream, args);
}

/* ------------------------------------------------------------------ GEMV chain */

/* The kernel's ChainOp (amdc_kernels.hip): 64 bytes. */
typedef struct {
  uint32_t type, sync, rows, nb, L, pad;
  const void *a;
  void *b;
  float *y;
  const float *bias, *res;
} chain_dev_op;
typedef char chain_dev_op_is_64_bytes[sizeof(chain_dev_op) == 64 ? 1 : -1];

typedef struct {
  chain_dev_op *ops; /* device: the list, then the barrier state (CHAIN_SYNC_BYTES) */
  uint32_t *sync;
  uint32_t n, grid, lds, nt, outb, vecb;
  uint64_t *trace; /* amdc_chain_trace's buffer (streaming form), or NULL */
  int k; /* the kernel: K_CHAIN, or K_CHAIN_S (+ 1 for Q4_K) for the streaming form */
} chain_t;

/* Threads per workgroup of the streaming chain (amdc_chain_s_*: one workgroup per CU): 4 staging
   and 8 compute waves. */
#define CHAIN_S_NT 768u
#define CHAIN_S_NC 8u

#define CHAIN_SPIN_NS 200000000u
#define CHAIN_SYNC_BYTES (35u * 128u) /* the kernel's NGRP + 3 lines */

/* A byte range [lo, hi) of device memory. */
typedef struct {
  uintptr_t lo, hi;
} span;
static span span_of(const void *p, u64 n) {
  span r = {(uintptr_t)p, (uintptr_t)p + (p ? (uintptr_t)n : 0u)};
  return r;
}
static int spans_meet(span a, span b) { return a.lo < a.hi && b.lo < b.hi && a.lo < b.hi && b.lo < a.hi; }
/* The bytes a (validated) chain operation writes (w[0], w[1]: an empty range where unused) and reads (r,
   returns how many ranges). */
static unsigned chain_spans(const amdc_chain_op *o, span *w, span r[4]) {
  if (o->type == AMDC_CHAIN_QUANT) { /* quantize: 32 nb floats -> 40 nb Q8 bytes */
    w[0] = span_of(o->q, 40ull * o->nb), w[1] = span_of(NULL, 0);
    r[0] = span_of(o->x, 128ull * o->nb);
    return 1;
  }
  if (o->type == AMDC_CHAIN_RMSNORM_Q8 || o->type == AMDC_CHAIN_SWIGLU_Q8) { /* RMSNorm (x, w -> y, q), SwiGLU (y, x -> y, q) */
    w[0] = span_of(o->y, 128ull * o->nb);
    w[1] = span_of(o->q, 40ull * o->nb);
    r[0] = span_of(o->x, 128ull * o->nb);
    r[1] = span_of(o->type == AMDC_CHAIN_RMSNORM_Q8 ? o->w : NULL, 128ull * o->nb);
    return 2;
  }
  w[0] = span_of(o->y, 4ull * o->rows), w[1] = span_of(NULL, 0);
  r[0] = o->type == AMDC_CHAIN_GEMV_X ? span_of(o->x, 128ull * o->nb) : span_of(o->xq, 40ull * o->nb);
  r[1] = span_of(o->w, (u64)o->rows * amdc_row_bytes_k(o->kind, o->nb));
  r[2] = span_of(o->bias, 4ull * o->rows);
  r[3] = span_of(o->res, 4ull * o->rows);
  return 4;
}

/* Two operations that may not run concurrently: one writes bytes the other reads or writes. */
static int chain_clash(const amdc_chain_op *a, const amdc_chain_op *b) {
  span wa[2], wb[2], ra[4], rb[4];
  const unsigned na = chain_spans(a, wa, ra), nb = chain_spans(b, wb, rb);
  int clash = 0;
  for (unsigned i = 0; i < 2u; i++) {
    for (unsigned j = 0; j < 2u; j++) clash |= spans_meet(wa[i], wb[j]);
    for (unsigned j = 0; j < na; j++) clash |= spans_meet(ra[j], wb[i]);
    for (unsigned j = 0; j < nb; j++) clash |= spans_meet(rb[j], wa[i]);
  }
  return clash;
}

int amdc_chain_create(const amdc_chain_op *ops, uint32_t n, void **chain) { return amdc_chain_create_form(ops, n, AMDC_CHAIN_AUTO, chain); }

int amdc_chain_create_form(const amdc_chain_op *ops, uint32_t n, int form, void **chain) {
  NEED_OPEN();
  if (form < AMDC_CHAIN_AUTO || form > AMDC_CHAIN_STREAMING) return fail(AMDC_EINVAL, "chain_create: form %d", form);
  if (!ops || !n || !chain) return fail(AMDC_EINVAL, "chain_create: null pointer or empty list");
  chain_dev_op *d = (chain_dev_op *)calloc(n, sizeof(chain_dev_op));
  if (!d) return fail(AMDC_EINVAL, "chain_create: out of host memory");
  u32 lds = 0, seg0 = 0;
  int rc = AMDC_OK;
  for (u32 k = 0; k < n && !rc; k++) {
    const amdc_chain_op *o = &ops[k];
    chain_dev_op *e = &d[k];
    e->sync = o->sync ? 1u : 0u, e->nb = o->nb;
    if (o->type == AMDC_CHAIN_QUANT) {
      if (!o->x || !o->q || !o->nb) rc = fail(AMDC_EINVAL, "chain op %u: quantize needs x, q and nb", k);
      else if (!aligned16(o->x)) rc = fail(AMDC_EINVAL, "chain op %u: x must be 16-byte aligned", k);
      e->type = 0, e->a = o->x, e->b = o->q;
    } else if (o->type == AMDC_CHAIN_GEMV || o->type == AMDC_CHAIN_GEMV_X) {
      const int fq = o->type == AMDC_CHAIN_GEMV_X; /* the f32 vector, quantized by every workgroup */
      const int k8 = o->kind == AMDC_KIND_Q8_0 || o->kind == AMDC_KIND_Q6_K;
      const u32 ng = amdc_ngroups(o->nb), need = (o->kind == AMDC_KIND_Q6_K ? 352u : 320u) * ng;
      rc = check_mat("chain gemv", o->kind, o->w, fq ? (const uint8_t *)o->x : o->xq, o->y, o->rows, o->nb);
      if (!rc && fq && k8) rc = fail(AMDC_EINVAL, "chain op %u: the f32-input GEMV takes Q4_0 and Q4_K (quantize Q8_0 / Q6_K inputs first)", k);
      if (!rc && k8 && (u64)o->rows * amdc_row_bytes_k(o->kind, o->nb) + amdc_row_bytes_k(o->kind, o->nb) >= (1ull << 32))
        rc = fail(AMDC_EINVAL, "chain op %u: the matrix must be under 4 GiB", k);
      if (!rc && need > GEMV_LDS_T1) rc = fail(AMDC_EINVAL, "chain op %u: nb %u too large", k, o->nb);
      if (k8) {
        /* the lanes per row of the decode launch (gemv_k8_launch) */
        e->type = o->kind == AMDC_KIND_Q6_K ? 6u : 5u, e->L = gemv2_lanes(ng, o->rows, 1);
      } else {
        e->type = (o->kind == AMDC_KIND_Q4_K ? 2u : 1u) + (fq ? 2u : 0u), e->L = gemv_lanes(ng);
      }
      e->rows = o->rows, e->a = o->w, e->b = fq ? (void *)o->x : (void *)o->xq, e->y = o->y, e->bias = o->bias, e->res = o->res;
      if (!rc && need > lds) lds = need;
    } else if (o->type == AMDC_CHAIN_RMSNORM_Q8 || o->type == AMDC_CHAIN_SWIGLU_Q8) {
      const int rn = o->type == AMDC_CHAIN_RMSNORM_Q8;
      if (!o->x || !o->y || !o->nb || (rn && !o->w))
        rc = fail(AMDC_EINVAL, "chain op %u: %s needs x, y%s and nb", k, rn ? "rmsnorm" : "swiglu", rn ? ", w" : "");
      else if ((u64)o->nb * 128u >= (1ull << 31)) rc = fail(AMDC_EINVAL, "chain op %u: nb %u too large", k, o->nb);
      else if (rn && !(o->eps >= 0.0f)) rc = fail(AMDC_EINVAL, "chain op %u: eps must be >= 0", k);
      else if (!rn && o->y == o->x) rc = fail(AMDC_EINVAL, "chain op %u: swiglu's x and y must differ", k);
      float eps = rn ? o->eps : 0.0f;
      e->type = rn ? 7u : 8u, e->a = o->x, e->b = o->q, e->y = o->y, e->bias = rn ? (const float *)o->w : NULL;
      memcpy(&e->pad, &eps, 4);
    } else {
      rc = fail(AMDC_EINVAL, "chain op %u: type %d", k, o->type);
    }
    /* two operations of one segment (no sync between) run concurrently: neither may write bytes
       the other reads or writes */
    for (u32 j = seg0; j < k && !rc; j++) {
      if (chain_clash(&ops[k], &ops[j])) rc = fail(AMDC_EINVAL, "chain op %u and op %u share bytes one of them writes, without a sync between them", k, j);
    }
    if (o->sync) seg0 = k + 1u;
  }
  if (rc) {
    free(d);
    return rc;
  }
  /* The streaming form (amdc_chain_s_*) runs lists whose GEMVs are all Q4_0 or all Q4_K, with at
     least one GEMV (the form AMDC_CHAIN_AUTO picks it for them). */
  u32 kinds = 0, ngemv = 0;
  for (u32 k = 0; k < n; k++) {
    if (d[k].type == 0u) continue;
    if (d[k].type >= 7u) { /* a producer operation: the persistent form only */
      kinds |= 8u;
      continue;
    }
    ngemv++;
    kinds |= d[k].type == 1u || d[k].type == 3u ? 1u : d[k].type == 2u || d[k].type == 4u ? 2u : 4u;
  }
  const int can_stream = ngemv && (kinds == 1u || kinds == 2u);
  if (form == AMDC_CHAIN_STREAMING && !can_stream) {
    free(d);
    return fail(AMDC_EINVAL, "chain_create: the streaming form needs at least one GEMV, every GEMV Q4_0 or every one Q4_K, and no producer operation");
  }
  const int streaming = form == AMDC_CHAIN_STREAMING || (form == AMDC_CHAIN_AUTO && can_stream);
  const int kk = streaming ? K_CHAIN_S + (kinds == 2u ? 1 : 0) : K_CHAIN;
  const u32 nt = streaming ? CHAIN_S_NT : 256u, cus = (u32)(g_cus > 0 ? g_cus : 256);
  u32 outb = 0, vecb = 0;
  if (streaming) {
    /* LDS of the streaming kernel: the workgroup's results of one operation (its 8 compute waves x
       their most row groups x rows per group, floats), then the vector */
    const u32 GW = CHAIN_S_NC * cus;
    u32 xrb = 0; /* the raw f32 vector of an f32-input operation */
    for (u32 k = 0; k < n; k++) {
      if (d[k].type == 0u) continue;
      const u32 rpw = 64u / d[k].L, nwr = (d[k].rows + rpw - 1u) / rpw, mj = (nwr + GW - 1u) / GW;
      if (4u * CHAIN_S_NC * mj * rpw > outb) outb = 4u * CHAIN_S_NC * mj * rpw;
      if (d[k].type >= 3u && 128u * d[k].nb > xrb) xrb = 128u * d[k].nb;
    }
    vecb = lds;
    lds += outb + xrb;
    if (lds > GEMV_LDS_T1) {
      free(d);
      return fail(AMDC_EINVAL, "chain_create: %u operations and their results need %u bytes of LDS in the streaming form", n, lds);
    }
  }
  int occ = 0;
  if (H.OccupancyMaxActiveBlocks(&occ, g_k[kk], (int)nt, lds) != 0 || occ < 1) {
    free(d);
    return fail(AMDC_EHIP, "chain_create: the chain kernel does not fit on a CU (LDS %u)", lds);
  }
  chain_t *c = (chain_t *)calloc(1, sizeof(chain_t));
  if (!c) {
    free(d);
    return fail(AMDC_EINVAL, "chain_create: out of host memory");
  }
  c->n = n, c->lds = lds, c->k = kk, c->nt = nt, c->outb = outb, c->vecb = vecb;
  c->grid = cus * (u32)(streaming ? 1 : occ < 2 ? occ : 2);
  const size_t bytes = (size_t)n * sizeof(chain_dev_op) + CHAIN_SYNC_BYTES;
  if (H.Malloc((void **)&c->ops, bytes) != 0) rc = fail(AMDC_EHIP, "chain_create: device allocation of %zu bytes", bytes);
  if (!rc) {
    c->sync = (uint32_t *)(c->ops + n);
    if (H.Memcpy(c->ops, d, (size_t)n * sizeof(chain_dev_op), hipMemcpyHostToDevice) != 0 ||
        H.Memset(c->sync, 0, CHAIN_SYNC_BYTES) != 0)
      rc = fail(AMDC_EHIP, "chain_create: upload");
  }
  free(d);
  if (rc) {
    if (c->ops) H.Free(c->ops);
    free(c);
    return rc;
  }
  *chain = c;
  return AMDC_OK;
}

int amdc_chain_launch(void *chain, void *stream) {
  NEED_OPEN();
  chain_t *c = (chain_t *)chain;
  if (!c) return fail(AMDC_EINVAL, "chain_launch: null chain");
  u32 spin = CHAIN_SPIN_NS;
  void *args[] = {&c->ops, &c->n, &c->sync, &spin, &c->outb, &c->vecb, &c->trace}; /* the streaming kernel's last three */
  if (c->k == K_CHAIN) args[4] = NULL;
  return launch_nt(c->k, c->grid, 1, c->nt, c->lds, stream, args);
}

int amdc_chain_trace(void *chain, uint64_t *buf) {
  NEED_OPEN();
  chain_t *c = (chain_t *)chain;
  if (!c) return fail(AMDC_EINVAL, "chain_trace: null chain");
  if (buf && c->k == K_CHAIN) return fail(AMDC_EINVAL, "chain_trace: the persistent form records no timeline");
  c->trace = buf;
  return AMDC_OK;
}

uint32_t amdc_chain_trace_words(void *chain) {
  const chain_t *c = (const chain_t *)chain;
  return c && c->k != K_CHAIN ? c->grid * (2u + 4u * c->n + 64u) : 0u;
}

int amdc_chain_check(void *chain) {
  NEED_OPEN();
  chain_t *c = (chain_t *)chain;
  if (!c) return fail(AMDC_EINVAL, "chain_check: null chain");
  HIPCALL(H.DeviceSynchronize());
  uint32_t st[CHAIN_SYNC_BYTES / 4u];
  HIPCALL(H.Memcpy(st, c->sync, CHAIN_SYNC_BYTES, hipMemcpyDeviceToHost));
  int dirty = 0;
  for (u32 i = 0; i < CHAIN_SYNC_BYTES / 4u; i++) dirty |= st[i] != 0u;
  if (dirty) {
    HIPCALL(H.Memset(c->sync, 0, CHAIN_SYNC_BYTES));
    return fail(AMDC_EHIP, "chain: a launch aborted at a grid barrier (abort flag %u, released barrier %u): not all %u workgroups were resident",
                st[34u * 32u], st[33u * 32u], c->grid);
  }
  return AMDC_OK;
}

int amdc_chain_destroy(void *chain) {
  NEED_OPEN();
  chain_t *c = (chain_t *)chain;
  if (!c) return AMDC_OK;
  HIPCALL(H.Free(c->ops));
  free(c);
  return AMDC_OK;
}

/* The recorder: amdc_chain_record_begin(stream) turns it on; the recordable operators called on that
 * stream then append to the list (rec_put) and launch nothing; amdc_chain_record_end builds the chain.
 * A grid barrier goes after an operation exactly when the next one shares bytes that one of them
 * writes with an operation since the last barrier (the rule amdc_chain_create checks), so independent
 * operations run concurrently, as the reference's megakernel joins independent GEMVs. */
static int rec_put(const amdc_chain_op *o) {
  if (g_rec.n == g_rec.cap) {
    const u32 cap = g_rec.cap ? 2u * g_rec.cap : 64u;
    amdc_chain_op *p = (amdc_chain_op *)realloc(g_rec.ops, (size_t)cap * sizeof *p);
    if (!p) {
      g_rec.err = 1;
      return fail(AMDC_EINVAL, "chain_record: out of host memory");
    }
    g_rec.ops = p, g_rec.cap = cap;
  }
  for (u32 j = g_rec.seg0; j < g_rec.n; j++)
    if (chain_clash(o, &g_rec.ops[j])) {
      g_rec.ops[g_rec.n - 1u].sync = 1;
      g_rec.seg0 = g_rec.n;
      break;
    }
  g_rec.ops[g_rec.n] = *o;
  g_rec.ops[g_rec.n].sync = 0;
  g_rec.n++;
  return AMDC_OK;
}

int amdc_chain_record_begin(void *stream) {
  NEED_OPEN();
  if (g_rec.on) return fail(AMDC_EINVAL, "chain_record_begin: a recording is already on");
  g_rec.on = 1, g_rec.stream = stream, g_rec.n = 0, g_rec.seg0 = 0, g_rec.err = 0;
  return AMDC_OK;
}

int amdc_chain_record_end(void *stream, int form, void **chain) {
  NEED_OPEN();
  if (!g_rec.on || stream != g_rec.stream) return fail(AMDC_EINVAL, "chain_record_end: no recording on this stream");
  g_rec.on = 0;
  if (!chain) return fail(AMDC_EINVAL, "chain_record_end: chain is NULL");
  *chain = NULL;
  if (g_rec.err) return fail(AMDC_EINVAL, "chain_record_end: an operator was refused while recording; no chain");
  if (!g_rec.n) return fail(AMDC_EINVAL, "chain_record_end: nothing was recorded");
  return amdc_chain_create_form(g_rec.ops, g_rec.n, form, chain);
}

/* ---------------------------------------------------------------- the streaming matrix load */

AMDC_HIDDEN int amdc_gguf_repack_rows(const amdc_gguf_tensor *t, const amdc_mat *m, u32 r0, u32 r1, int nthreads, uint8_t *dst);
AMDC_HIDDEN int amdc_gguf_tensor_ptr(const amdc_gguf *g, const char *name, const amdc_gguf_tensor **t);


/* The two pinned staging buffers of the load and their events, kept for
 * later loads (pinning memory costs milliseconds), freed by amdc_close. */
static void *g_stg[2];
static hipEvent_t g_stg_ev[2];
static size_t g_stg_bytes;

static int stage_reserve(size_t n) {
  if (n <= g_stg_bytes && g_stg[0]) return AMDC_OK;
  for (int b = 0; b < 2; b++) {
    if (g_stg[b]) H.HostFree(g_stg[b]);
    g_stg[b] = NULL;
  }
  g_stg_bytes = 0;
  hipError_t e;
  for (int b = 0; b < 2; b++) {
    if ((e = H.HostMalloc(&g_stg[b], n, 0))) return fail(AMDC_EHIP, "gguf_load: pinned staging of %zu bytes: %s", n, H.GetErrorString(e));
    if (!g_stg_ev[b] && (e = H.EventCreate(&g_stg_ev[b]))) return fail(AMDC_EHIP, "gguf_load: %s", H.GetErrorString(e));
  }
  g_stg_bytes = n;
  return AMDC_OK;
}

static void stage_free(void) {
  for (int b = 0; b < 2; b++) {
    if (g_stg[b]) H.HostFree(g_stg[b]);
    if (g_stg_ev[b]) H.EventDestroy(g_stg_ev[b]);
    g_stg[b] = NULL, g_stg_ev[b] = NULL;
  }
  g_stg_bytes = 0;
}

/* Chunks of rows alternate between two pinned staging buffers: chunk c is
 * repacked into buffer c & 1 once the copy of chunk c - 2 out of it has
 * finished (its event), then copied with hipMemcpyAsync on the stream, so the
 * repack of one chunk runs while the previous one crosses PCIe. */
int amdc_gguf_load(const amdc_gguf *g, const char *name, int nthreads, amdc_mat *m, void *stream) {
  NEED_OPEN();
  int rc = amdc_gguf_mat_info(g, name, m);
  const amdc_gguf_tensor *t = NULL;
  if (!rc) rc = amdc_gguf_tensor_ptr(g, name, &t);
  if (rc) return rc;
  const u64 rb = m->bytes / m->rows;
  /* bytes of repacked rows per staging buffer: 32 MiB (AMDC_LOAD_CHUNK_KB) */
  const u64 chunk = (u64)envi("AMDC_LOAD_CHUNK_KB", 32768) << 10;
  u32 per = (u32)(chunk / rb);
  if (per < 1u) per = 1u;
  if (per > m->rows) per = m->rows;
  void *dev = NULL, *stg[2];
  int used[2] = {0, 0};
  hipError_t e = H.Malloc(&dev, m->bytes);
  if (e) return fail(AMDC_EHIP, "gguf_load: hipMalloc of %llu bytes: %s", (unsigned long long)m->bytes, H.GetErrorString(e));
  if ((rc = stage_reserve((size_t)per * rb))) {
    H.Free(dev);
    return rc;
  }
  stg[0] = g_stg[0], stg[1] = g_stg[1];
  for (u32 r0 = 0, c = 0; !rc && r0 < m->rows; r0 += per, c++) {
    const u32 r1 = m->rows - r0 < per ? m->rows : r0 + per, b = c & 1u;
    if (used[b] && (e = H.EventSynchronize(g_stg_ev[b]))) {
      rc = fail(AMDC_EHIP, "gguf_load: %s", H.GetErrorString(e));
      break;
    }
    if ((rc = amdc_gguf_repack_rows(t, m, r0, r1, nthreads, (uint8_t *)stg[b]))) break;
    if ((e = H.MemcpyAsync((uint8_t *)dev + (u64)r0 * rb, stg[b], (size_t)(r1 - r0) * rb, hipMemcpyHostToDevice, stream)) ||
        (e = H.EventRecord(g_stg_ev[b], stream)))
      rc = fail(AMDC_EHIP, "gguf_load: copy: %s", H.GetErrorString(e));
    used[b] = 1;
  }
  for (int b = 0; b < 2; b++) /* every copy out of the staging buffers is done before the next use */
    if (used[b] && (e = H.EventSynchronize(g_stg_ev[b])) && !rc) rc = fail(AMDC_EHIP, "gguf_load: %s", H.GetErrorString(e));
  if (rc) {
    H.Free(dev);
    return rc;
  }
  m->w = dev;
  return AMDC_OK;
}

int amdc_mat_release(amdc_mat *m) {
  if (!m) return fail(AMDC_EINVAL, "mat_release: null");
  if (m->w) {
    NEED_OPEN();
    HIPCALL(H.Free(m->w));
  }
  m->w = NULL;
  return AMDC_OK;
}
