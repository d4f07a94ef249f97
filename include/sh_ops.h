/* softhier-ops for MI355X (gfx950): the C ABI.
 *
 * This header re-exports the hot-path subset of the reference's operator library header
 * (runwangdl/softhier-mlir runtime/sh_ops.h) with the same names, argument order, types and error codes,
 * so the same op sequence (emitted programs, C test drivers, ctypes callers) runs unchanged. Each
 * declaration cites the reference line it replaces.
 *
 * Execution model (differs from the reference's SPMD model, same observable results):
 *  - One host thread calls each op once. The op validates its arguments on the host, then enqueues HIP
 *    kernels on the library stream (sh_set_stream; default: the legacy null stream, which is ordered with
 *    PyTorch's default stream). Ops are stream-ordered and asynchronous; sh_barrier_global() drains them.
 *  - Tensors are fp16 row-major in GPU memory, addressed by 64-bit byte addresses (device pointers:
 *    a torch tensor's data_ptr(), sh_hbm_addr() or sh_hbm_malloc()). Leading dimensions are in elements.
 *  - `cluster` is accepted for source compatibility and ignored: the op always runs on the whole GPU.
 *    sh_cluster_id() == 0, sh_is_first_core() == 1 and sh_num_clusters() == 1, so guards such as
 *    `if (sh_cluster_id() == 0 && sh_is_first_core())` in emitted code fire exactly once.
 *  - Constraint checks mirror the reference (same conditions, same return codes, same budgets: the
 *    reference's 1 MiB cluster TCDM, reported by sh_l1_size()), so a call fails here exactly when it
 *    fails there. The additive entry points at the end carry no TCDM budget.
 *  - A HIP runtime failure makes an int op return SH_EHIP (-3, additive) and records the message
 *    (sh_last_error / sh_last_error_str); void ops record it the same way.
 *  - Not re-entrant across host threads.
 */
#ifndef SH_OPS_H
#define SH_OPS_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime wrappers (reference runtime/sh_ops.h:19-37, runtime/sh_rt.inc.c:2-29) ---------------------- */
void     sh_init(void);                 /* sh_ops.h:20   picks up the current HIP device; idempotent */
void     sh_barrier_global(void);       /* sh_ops.h:21   drains the library stream */
void     sh_barrier_cluster(void);      /* sh_ops.h:22   same as sh_barrier_global */
uint32_t sh_cluster_id(void);           /* sh_ops.h:23   0 */
uint32_t sh_core_id(void);              /* sh_ops.h:24   0 */
int      sh_is_first_core(void);        /* sh_ops.h:25   1 */
int      sh_is_dm_core(void);           /* sh_ops.h:26   1 */
uint32_t sh_num_clusters(void);         /* sh_ops.h:27   1: the GPU is one cluster */
void     sh_timer_start(void);          /* sh_ops.h:28   HIP event on the library stream */
void     sh_timer_end(void);            /* sh_ops.h:29   prints "[Performance Counter]: Execution period is N ns", restarts */
void     sh_eoc(uint32_t val);          /* sh_ops.h:30   drains the stream, flushes stdout, records val */
uint32_t sh_cycles(void);               /* sh_ops.h:31   ns since sh_init (1 GHz equivalence), read after the stream drains */
void     sh_printf(const char *fmt, ...);                /* sh_ops.h:32 */
uint64_t sh_hbm_addr(uint64_t byte_offset);             /* sh_ops.h:33   arena base + offset (arena: SH_HBM_ARENA_BYTES, default 1 GiB, lazy) */
uint64_t sh_hbm_malloc(uint32_t bytes);                 /* sh_ops.h:34   separate device allocation, 256 B aligned */
uint32_t sh_l1_size(void);                              /* sh_ops.h:35   the reference cluster's TCDM bytes (0x100000) */
void     sh_preload_wait(uint64_t sentinel);            /* sh_ops.h:36   drains the stream (data is resident) */
/* Additive: copy the PT_LOAD segments of a preload image (ELF32, softhier_mlir/sim/preload.py:38-78: segment at
 * physical address SH_PRELOAD_HBM_BASE + offset) into the sh_hbm_addr arena at those offsets. Returns the number of
 * segments copied, -1 for an unreadable / malformed image or a segment beyond the arena, SH_EHIP on a HIP failure. */
#define SH_PRELOAD_HBM_BASE 0xC0000000u
int      sh_preload_load(const char *path);
void     sh_call_on_core_stack(void (*fn)(void), uint32_t bytes_per_core);   /* sh_ops.h:48   calls fn() */

#define SH_ALL 0xFFFFFFFFu                              /* sh_ops.h:39 */
#define SH_CORE_STACK_BYTES 40960u                      /* sh_ops.h:47 */
#define SH_SELF (sh_cluster_id())                       /* sh_ops.h:308 */

/* ---- formats (sh_ops.h:51) -------------------------------------------------------------------------- */
enum sh_fmt { SH_FP16 = 0, SH_FP8 = 1, SH_INT16 = 2, SH_INT8 = 3 };

/* ---- GEMM: Z[M,N] (+)= X[M,K] . W[K,N] (sh_ops.h:53-88, runtime/sh_gemm.inc.c:12-189) ------------------
 * fp16 operands, fp32 accumulation on MFMA, fp16 result (RNE). tm/tn/tk are the caller's tile hints: they set
 * the divisibility rule exactly as in the reference (0 -> 256); the GPU tile is chosen by the library. */
typedef struct {
    uint32_t tm, tn, tk;     /* tile; 0 -> 256 */
    uint32_t pipeline;       /* accepted (the GPU kernels always double-buffer) */
    uint32_t accumulate;     /* 1: Z += X.W (Z read first); 0: Z = X.W */
    uint32_t fmt;            /* enum sh_fmt; only SH_FP16 computes (others: -1) */
    uint32_t l1_base;        /* counts towards the TCDM budget exactly as in the reference */
} sh_gemm_cfg;               /* sh_ops.h:54-60 */

/* sh_ops.h:66-67 (sh_gemm.inc.c:53-117): -1 when M%tm, N%tn or K%tk != 0 (or fmt != SH_FP16, or a NULL
 * address), -2 when sh_gemm_l1_bytes() exceeds the reference TCDM, SH_EHIP on a HIP failure, else 0. */
int sh_gemm(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
            uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, uint32_t cluster);

/* sh_ops.h:72-73 (sh_gemm.inc.c:127-189): SUMMA mode over a virtual SH_MESH_P x SH_MESH_P mesh of output
 * tiles (the reference's 4 x 4 cluster mesh). Same constraints and codes: tm == tn, M == N == P * tm,
 * K % tk == 0 (-1), TCDM budget (-2). The launch is the tiled GEMM with its XCD-aware tile order (each XCD
 * walks a contiguous band of output tile rows, so an X row panel is fetched into one XCD's L2 and re-read there
 * by the whole band); there is no separate mesh schedule and no broadcast step on one GPU. */
#define SH_MESH_P 4u
int sh_gemm_mesh(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                 uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg);

/* sh_ops.h:88 (sh_gemm.inc.c:24-30): l1_base + (pipeline ? 2 : 1) * (tm*tk + tk*tn) * 2 + tm*tn*2. */
uint32_t sh_gemm_l1_bytes(uint32_t M, uint32_t N, uint32_t K, const sh_gemm_cfg *cfg);

/* Small-M GEMM (sh_ops.h:74-85): Z = X.W (+= with cfg->accumulate) with the reference's plan checks. cfg fields
 * are "0 = auto" here: tm = rows per block (must divide M), tn = column granule (4), tk = K panel. Returns 0, -1
 * (tm does not divide M / NULL), -2 (no plan fits the reference's scratch limit 0x90000 from l1_base), -3 (fmt). */
enum { SH_XM_AUTO = 0, SH_XM_PANEL = 1, SH_XM_WHOLE = 2 };                                   /* sh_ops.h:79 */
int sh_gemm_xmcast(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                   uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg);        /* sh_ops.h:80-81 */
int sh_gemm_xmcast_ex(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                      uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, uint32_t mode);  /* sh_ops.h:82-83 */
uint32_t sh_gemm_xmcast_l1_bytes(uint32_t M, uint32_t N, uint32_t K, const sh_gemm_cfg *cfg, uint32_t mode);  /* sh_ops.h:84, ~0u: no plan */

/* ---- row-wise / elementwise ops (sh_ops.h:90-100, runtime/sh_rowops.inc.c:383-465) -------------------
 * fp16 in/out, one pass over HBM. Parameter rows (gamma, beta, bias) are fp16 rows. LayerNorm, softmax and
 * scale compute in fp32; add / add_bias use packed fp16 adds (which round exactly as the fp32 sum rounded to
 * fp16); GELU is the tanh form evaluated on packed fp16 (a few fp16 ulps from the fp32 form). */
void sh_layernorm(uint64_t y, uint64_t x, uint64_t gamma, uint64_t beta, uint32_t rows, uint32_t cols, uint32_t ld, float eps, uint32_t cluster);  /* sh_ops.h:94 */
void sh_softmax_rows(uint64_t y, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, float scale, uint32_t cluster);  /* sh_ops.h:95 */
void sh_gelu(uint64_t y, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t cluster);                     /* sh_ops.h:96 tanh form */
void sh_add(uint64_t y, uint64_t a, uint64_t b, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t cluster);          /* sh_ops.h:97 */
void sh_add_bias(uint64_t y, uint64_t x, uint64_t bias_row, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t cluster); /* sh_ops.h:98 */
void sh_scale(uint64_t y, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, float s, uint32_t cluster);           /* sh_ops.h:99 */
void sh_transpose(uint64_t dst, uint64_t src, uint32_t rows, uint32_t cols, uint32_t ld_src, uint32_t ld_dst, uint32_t cluster); /* sh_ops.h:100 bit-exact */
/* No counterpart in the reference (LayerNorm folded into the next GEMM, sh_gemm_epi.ln_stats): per row of x, the
 * mean and 1 / sqrt(biased variance + eps) as fp32 pairs into stats [rows][2], the statistics sh_layernorm
 * computes (two passes over the row in fp32). */
void sh_row_stats(uint64_t stats, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, float eps);
/* No counterpart in the reference: the weight side of the fold for z = LN(x) . W + b, W [K, N] (ldw):
 * wp = r16(gamma_k W[k][n]) (fp16, leading dim ldwp), c[n] = sum_k wp[k][n] (fp32), d[n] = sum_k beta_k W[k][n]
 * + b[n] (fp32; bias = 0: none). gamma, beta, bias: fp16 rows. Run once per weight. */
void sh_ln_fold(uint64_t wp, uint64_t c, uint64_t d, uint64_t w, uint64_t gamma, uint64_t beta, uint64_t bias,
                uint32_t K, uint32_t N, uint32_t ldw, uint32_t ldwp);
/* sh_ops.h:218 (sh_l1.inc.c:58-61): 1-D copy of `bytes` from src to dst in HBM (non-overlapping), enqueued on the
 * library stream (the reference's call is synchronous on its DM core; here it is ordered like every other op). */
void sh_dma_copy(uint64_t dst, uint64_t src, uint32_t bytes);
/* No counterpart in the reference: read [addr, addr + bytes) through the GPU's caches (L2 and the 256 MB Infinity
 * Cache) on the library stream, writing nothing, so that a kernel launched later finds those bytes cached instead of
 * in HBM. For callers that know which weights come next: the encoder stack issues it on a second stream for a
 * layer's remaining weights while its attention runs. 0, -1 for a NULL address, SH_EHIP for a launch failure. */
int sh_prefetch(uint64_t addr, uint64_t bytes);

/* ---- fused attention (sh_ops.h:102-127, runtime/sh_attention.inc.c:55-243) ----------------------------
 * o = softmax(scale * q k^T) v per head; head h = columns [h*dh, (h+1)*dh). Flash-style on the GPU (online
 * softmax over key blocks, scores never leave the CU), so sq only has to satisfy the reference's rules. */
int sh_attention_head(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t dh,
                      uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint32_t cluster);   /* sh_ops.h:109-110 */
int sh_attention_q(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t D, uint32_t H,
                   uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint32_t cluster, uint32_t sq); /* sh_ops.h:114-115 */
int sh_attention(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t D, uint32_t H,
                 uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint32_t cluster);      /* sh_ops.h:116-117 */
uint32_t sh_attention_l1_bytes_q(uint32_t S, uint32_t dh, uint32_t sq);   /* sh_ops.h:118 */
uint32_t sh_attention_l1_bytes(uint32_t S, uint32_t dh);                  /* sh_ops.h:119 */
uint32_t sh_attention_q_block(uint32_t S, uint32_t dh, uint32_t H, uint32_t P);   /* sh_ops.h:123 same rule */
/* sh_ops.h:127: ns stamps of the last attention call's last workgroup, from its first workgroup's start (phase 7
 * = 0): 0 start, 1-2 operands staged, 3-4 first key block's scores / row maximum known, 5 every key block done,
 * 6 stored (the kernels without stamps report only 6, the launch's event time; all 0 when that call was
 * sh_attention_batched or made under stream capture, which carry no stamps). */
uint32_t sh_attention_profile(uint32_t S, uint32_t dh, uint32_t phase);

/* ---- Llama-style decoder ops (sh_ops.h:277-307, runtime/sh_llm.inc.c) -----------------------------------
 * Token masks: tok[j] (uint16, one per position) is the cumulative attention-block id of position j, SH_LLM_PAD
 * for padding; query i attends key j iff tok[j] <= tok[i] (unsigned). A padding query row (or one with no allowed
 * key) is uniform. Row ops need cols % 4 == 0 (and cols <= 8192 here); violations set sh_last_error and return. */
#define SH_LLM_PAD 0xFFFFu                                                                         /* sh_ops.h:283 */
void sh_rmsnorm(uint64_t y, uint64_t x, uint64_t gamma, uint32_t rows, uint32_t cols, uint32_t ld, float eps, uint32_t cluster);  /* sh_ops.h:284 */
void sh_rope(uint64_t y, uint64_t x, uint64_t cos_sin, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t ld_table, uint32_t dh,
             uint32_t cluster);                                                                    /* sh_ops.h:288, rotate-half */
void sh_silu_mul(uint64_t y, uint64_t a, uint64_t b, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t cluster);  /* sh_ops.h:289 */
void sh_softmax_masked(uint64_t y, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, float scale, uint64_t tok_q,
                       uint64_t tok_k, uint32_t cluster);                                          /* sh_ops.h:292, scale > 0 */
int sh_attention_head_masked(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t dh, uint32_t ldq,
                             uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint64_t tok, uint32_t cluster);  /* sh_ops.h:294-295 */
int sh_attention_gqa(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t D, uint32_t H, uint32_t Hkv,
                     uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint64_t tok, uint32_t cluster);  /* sh_ops.h:299-300 */
void sh_pixel_shuffle(uint64_t dst, uint64_t src, uint32_t grid, uint32_t D, uint32_t s, uint32_t cluster);  /* sh_ops.h:303, bit-exact */

/* ---- test helpers (sh_ops.h:220-240, runtime/sh_test.inc.c, runtime/sh_rt.inc.c:31-59) ----------------
 * Fills run as GPU kernels (LCG jump-ahead per element, identical values to the sequential loop); dumps
 * gather on the GPU and print on the host in the reference's "<tag> r c hex" format. */
void sh_test_fill_int_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t seed, int lo, int hi);              /* sh_ops.h:223 */
void sh_test_fill_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t seed, int lo, int hi, float scale);     /* sh_ops.h:224 */
void sh_test_dump_samples(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t seed, uint32_t nsamples, const char *tag); /* sh_ops.h:226 */
void sh_test_dump_samples_idx(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t seed, uint32_t nsamples, const char *tag, uint32_t idx); /* sh_ops.h:227 */
uint32_t sh_test_check_gemm(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                            uint32_t ldx, uint32_t ldw, uint32_t ldz, uint32_t nsamples, float tol,
                            float z0, const char *tag);                                                                        /* sh_ops.h:230-232 */
void     sh_test_fill_const_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t bits);                        /* sh_ops.h:234 */
void     sh_test_fill_colparity_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t even, uint32_t odd);      /* sh_ops.h:235 */
uint32_t sh_test_check_const_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t bits, uint32_t tol, const char *tag); /* sh_ops.h:236 */
void sh_test_dump_all(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, const char *tag);                                  /* sh_ops.h:183 */
void sh_test_dump_all_idx(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, const char *tag, uint32_t idx);                /* sh_ops.h:184 */
float    sh_fp16_to_f32(uint16_t h);    /* sh_ops.h:239 IEEE binary16 -> binary32, exact */
uint16_t sh_f32_to_fp16(float f);       /* sh_ops.h:240 RNE; overflow -> Inf; NaN -> 0x7E00 | sign */

/* sh_ops.h:249-258 hardware register conversions: portable equivalents on the host (low 16 bits used). */
static inline float    sh_h2f(uint32_t h) { return sh_fp16_to_f32((uint16_t)(h & 0xFFFFu)); }
static inline uint32_t sh_f2h(float f)    { return 0xFFFF0000u | sh_f32_to_fp16(f); }

/* ====================================================================================================
 * Additive entry points (no counterpart in the reference's ABI; existing layouts are unchanged).
 * ==================================================================================================== */
#define SH_EHIP (-3)                     /* an int op's return code for a HIP runtime failure */

int         sh_last_error(void);         /* 0, or the code of the last failure (-1 args, SH_EHIP HIP); cleared on read */
const char *sh_last_error_str(void);     /* message of the last failure ("" if none) */
void        sh_set_stream(uint64_t stream);   /* hipStream_t to enqueue on (0 = legacy null stream) */
uint64_t    sh_get_stream(void);
/* Split-K calls keep an fp32 partials workspace per stream they ran on (at least 64 MiB each, grown geometrically,
 * outgrown buffers kept because graphs captured earlier may address them), so a caller that creates and destroys
 * streams would otherwise hold that memory until exit. sh_stream_release(stream) waits for the stream, then frees
 * everything the library holds for it (0, or SH_EHIP); the next split-K call on that stream allocates again. Call
 * it only when no graph captured on that stream will be replayed. sh_stream_workspace_bytes: the live workspace
 * of a stream (0 if none). */
int         sh_stream_release(uint64_t stream);
uint64_t    sh_stream_workspace_bytes(uint64_t stream);
double      sh_timer_last_ns(void);      /* the period sh_timer_end() printed last */
/* Text capture for in-process callers: while on, everything the library prints (sh_printf, sample dumps,
 * timer lines) is appended to an internal buffer instead of stdout. sh_captured copies it out (NUL
 * terminated, truncated to cap - 1) and returns its full length; turning capture on clears it. */
void        sh_capture(int on);
uint64_t    sh_captured(char *buf, uint64_t cap);

/* Split-K GEMM: K is cut into `splits` contiguous ranges computed by separate workgroups into an fp32
 * workspace owned by the library, then reduced in a fixed order (deterministic) and rounded once to fp16.
 * Two equal ranges (K % 128 == 0) run in one workgroup per tile instead, whose two halves add their fp32 sums
 * in that same order: the same bits, no workspace, no reduction launch.
 * Shape/tile checks as sh_gemm (-1/-2); splits == 0 lets the library choose. */
int sh_gemm_splitk(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                   uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, uint32_t splits, uint32_t cluster);

/* No counterpart in the reference: sh_gemm_splitk for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments, checks and results
 * (the same kernels and summation order, so the same bits); the fp32 partials live in a fixed 16 MiB array of
 * the library's code object on each GPU, so the call makes no hipMalloc / hipFree and skips the one-time tile
 * timing. Returns -1 (before any GPU work) when a launch that writes partials needs more than 16 MiB of them
 * (splits x M x N x 4 bytes); a request of two equal K ranges (K % 128 == 0, 16-byte aligned operands) runs both
 * ranges in one workgroup and writes none, at any size. All calls on one GPU share that array: calls that overlap
 * on one GPU race. */
int sh_gemm_splitk_noalloc(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                           uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, uint32_t splits, uint32_t cluster);

/* Fused GEMM epilogue: z = act(X.W [+ z_old if cfg->accumulate] + bias) rounded to fp16, then
 * [+ residual, rounded again]. bias: 0 or an fp16 (SH_BIAS_FP16) / fp32 (SH_BIAS_FP32) row of N values.
 * residual: 0 or an fp16 [M,N] tensor with leading dim ldr (may alias z). No tile-divisibility rule and no
 * TCDM budget; M, N, K >= 1. splits: as sh_gemm_splitk (1 = no split, 0 = library choice). */
enum { SH_ACT_NONE = 0, SH_ACT_GELU = 1 };
enum { SH_BIAS_FP16 = 0, SH_BIAS_FP32 = 1 };
typedef struct {
    uint64_t bias;        /* 0: none */
    uint32_t bias_fmt;    /* SH_BIAS_FP16 | SH_BIAS_FP32 */
    uint32_t act;         /* SH_ACT_NONE | SH_ACT_GELU (tanh form, as sh_gelu) */
    uint64_t residual;    /* 0: none */
    uint32_t ldr;         /* leading dim of residual (elements) */
    uint32_t splits;      /* 1: none; 0: library choice */
    /* LayerNorm folded into the GEMM (0: off). With X the raw rows and W' = diag(gamma) W, c = 1^T W' and
     * d = beta^T W + b from sh_ln_fold, the product p = X . W' becomes z = r p - r mu c + d before the rest of the
     * chain (act, residual), which is LN(X) . W + b; ln_stats: fp32 [M][2] (mu, r) rows from sh_row_stats (8-byte
     * aligned, else -1), ln_c: fp32 row of N, and the bias must then be the fp32 row d (SH_BIAS_FP32). Rounded once
     * to fp16. */
    uint64_t ln_stats;
    uint64_t ln_c;
    /* Row partials (0: off): the GEMM also writes, for each stored row of Z and each 32 columns of it, the fp32 pair
     * (sum s, M2 = sum (z - s / 32)^2) of the stored fp16 values to stats_out [M][N / 32] (N % 32 == 0, 16-byte
     * aligned operands): the statistics the next GEMM's LayerNorm fold needs, without a pass over Z. That GEMM
     * takes them with ln_stats = stats_out, ln_parts = N / 32 (its K / 32) and ln_eps, and forms mean and
     * variance with Chan's pairwise combination; ln_parts = 0: ln_stats holds (mean, r) rows of sh_row_stats. */
    uint64_t stats_out;
    uint32_t ln_parts;
    float ln_eps;
} sh_gemm_epi;
int sh_gemm_ex(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
               uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, const sh_gemm_epi *epi);

/* No counterpart in the reference: sh_gemm_ex with the weight given transposed, wt = W^T as an [N, K] row-major
 * tensor with leading dim ldwt >= K (z = X . W, W[k][n] = wt[n * ldwt + k]). For callers that keep their weights
 * transposed once (the encoder layer): both operands are then rows of k, which lets the GPU use larger tiles and
 * plain LDS reads. Same epilogue, checks and codes as sh_gemm_ex (-1 also for ldwt < K). */
int sh_gemm_ex_wt(uint64_t x, uint64_t wt, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                  uint32_t ldx, uint32_t ldwt, uint32_t ldz, const sh_gemm_cfg *cfg, const sh_gemm_epi *epi);

/* Additive (no counterpart in the reference): the GEMM cost model's plan for an (M, N, K) problem with
 * 16-byte-aligned operands and a split request (0 = library choice): out[0] tile configuration, out[1] /
 * out[2] its tile rows / columns, out[3] the split count. A large problem's first call may still replace the
 * configuration by its one-time timing. Runs no GPU work. 0, or -1 for an empty problem / NULL out. */
int sh_gemm_plan(uint32_t M, uint32_t N, uint32_t K, uint32_t splits, uint32_t *out);

/* Additive (no counterpart in the reference): the GEMM tile table that sh_gemm_plan indexes and SH_GEMM_CFG forces.
 * sh_gemm_tile_count: its entries. sh_gemm_tile_info(i, out): out[0] / out[1] tile rows / columns, out[2] kernel
 * family (1 register-staged: any alignment and K; 2 direct-to-LDS with a partial last k-slice variant; 5
 * direct-to-LDS, register epilogue; 6 direct-to-LDS for the W^T operand), out[3] threads per workgroup, out[4] W^T
 * operand, out[5] register epilogue (LayerNorm fold and row partials without fp32 partials), out[6] in-workgroup
 * split of two equal K ranges, out[7] partial-k-slice variant. Unsplit direct-to-LDS configurations (families 2, 5
 * and 6) store the same bits; the register-staged ones (1) store the same bits among themselves. 0, or -1 for i out
 * of range / NULL out. No GPU work. */
int sh_gemm_tile_count(void);
int sh_gemm_tile_info(uint32_t i, uint32_t *out);

/* Batched multi-head attention (the reference has no batch dimension): sequence b uses q + b*bsq*2 bytes,
 * likewise k/v/o with their own batch strides in elements (e.g. S*ld for rows stacked as [B*S, ld]).
 * Constraints as sh_attention_q except the TCDM budget; sq == 0 -> the library's choice. */
int sh_attention_batched(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t B, uint32_t S, uint32_t D, uint32_t H,
                         uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo,
                         uint64_t bsq, uint64_t bsk, uint64_t bsv, uint64_t bso, float scale, uint32_t sq);
/* No counterpart in the reference: sh_attention_batched that also reads two ranges [pfN, pfN + pfN_bytes) (bytes 0:
 * none) into the GPU's caches (L2 and the Infinity Cache) while it runs, writing nothing there: the same outputs, bit
 * for bit. For callers that know which weights the next kernels read (the encoder stack: a layer's out-proj and FFN
 * weights and the next layer's QKV weight, which do not all stay in the cache next to the activations); attention
 * leaves memory bandwidth and room on every CU, so the reads cost it little and no second stream or event is
 * needed. A head the one-pass kernel does not take reads the ranges after its kernel instead (sh_prefetch). -1 also
 * for a NULL range with bytes > 0. */
int sh_attention_batched_prefetch(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t B, uint32_t S, uint32_t D, uint32_t H,
                                  uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo,
                                  uint64_t bsq, uint64_t bsk, uint64_t bsv, uint64_t bso, float scale, uint32_t sq,
                                  uint64_t pf0, uint64_t pf0_bytes, uint64_t pf1, uint64_t pf1_bytes);

/* LayerNorm with separate input / output leading dims (fused residual stream layouts). */
void sh_layernorm_ld(uint64_t y, uint64_t x, uint64_t gamma, uint64_t beta, uint32_t rows, uint32_t cols,
                     uint32_t ldy, uint32_t ldx, float eps);

#ifdef __cplusplus
}
#endif
#endif /* SH_OPS_H */
