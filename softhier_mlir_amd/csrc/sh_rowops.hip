// Row-wise and elementwise fp16 ops (reference runtime/sh_rowops.inc.c:383-465, semantics of
// tests/gvsoc/run.py:152-158). Every op reads its inputs from HBM once and writes its output once:
//  - layernorm / softmax: one wavefront per row, the whole row held in registers as fp32 (16-byte loads),
//    statistics by wavefront butterfly reductions, then the output pass from registers;
//  - gelu / add / add_bias / scale: a flat grid over 16-byte chunks (8 halves per lane per access);
//  - transpose: 128 x 128 tiles, 8 x 8 register transposes into a swizzled LDS tile, 16-byte row stores;
//    pure 16-bit moves, so the result is bit-exact (NaN payloads included).
// Rows wider than the register-resident limit (8192 columns) use a block-per-row loop kernel. Tensors
// whose base, leading dim or width is not a multiple of 8 halves take element-wise variants.
#include "sh_common.h"
#include <algorithm>
#include <cstdlib>

namespace {

constexpr int kRowWaves = 4;          // rows per 256-thread block
enum { OP_GELU = 0, OP_ADD = 1, OP_BIAS = 2, OP_SCALE = 3, OP_SILU_MUL = 4 };

__device__ __forceinline__ void unpack8(const uint4 q, float *f) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = sh_dev_h2f((uint16_t)(w[i] & 0xFFFFu));
        f[2 * i + 1] = sh_dev_h2f((uint16_t)(w[i] >> 16));
    }
}
__device__ __forceinline__ uint4 pack8(const float *f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)sh_dev_f2h(f[2 * i]) | ((uint32_t)sh_dev_f2h(f[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Element index of slot (u, i) of a lane: vector layout = 8 consecutive halves per chunk, chunks strided by
// 64 lanes; scalar layout = one half per lane, strided by 64.
template <bool VEC>
__device__ __forceinline__ uint32_t slot_col(int lane, int u, int i) {
    return VEC ? 8u * (uint32_t)(lane + 64 * u) + (uint32_t)i : (uint32_t)lane + 64u * (uint32_t)(8 * u + i);
}

// 16-byte chunk u of a row for this lane: every chunk is loaded (one past the row end reads chunk 0 and is
// zeroed in unpack_row), so all the loads of a row are in flight together.
// Makes q's value available at this point (an empty asm that reads and writes it), so its load is not moved later.
__device__ __forceinline__ void pin4(uint4 &q) { __asm__ volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w)); }

// 16-byte store; nt: nontemporal (streaming), used when the output is at least half the 256 MB Infinity Cache: with
// its input it does not stay there, so no consumer could find it cached and plain stores only evict what it could
// use (at 16x the encoder's rows, ~200 MB outputs: LayerNorm 5.7 against 5.5 TB/s, add_bias 6.0 against 5.6).
typedef uint32_t sh_u4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st16(void *p, uint4 v, bool nt) {
    if (nt) __builtin_nontemporal_store((sh_u4v){v.x, v.y, v.z, v.w}, (sh_u4v *)p);
    else *(uint4 *)p = v;
}
constexpr uint64_t kNtBytes = uint64_t(128) << 20;     // half the MI355X Infinity Cache
// 16-byte load, nontemporal under NT: the kernels that stream a nontemporal output read their input once too, so
// its lines need not stay cached either (at 16x the encoder's rows: softmax, add and the copy +2-4 %, GELU, add_bias
// and transpose +2 %). LayerNorm keeps plain loads: its row groups walk rows with a stride, and nontemporal loads
// measured 8 % slower there.
template <bool NT>
__device__ __forceinline__ uint4 ld16(const void *p) {
    if constexpr (NT) {
        const sh_u4v q = __builtin_nontemporal_load((const sh_u4v *)p);
        return make_uint4(q.x, q.y, q.z, q.w);
    } else {
        return *(const uint4 *)p;
    }
}

template <int NCH>
__device__ __forceinline__ void load_raw(const uint16_t *__restrict__ p, uint32_t cols, int lane, uint4 (&raw)[NCH]) {
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
        const uint32_t c0 = slot_col<true>(lane, u, 0);
        raw[u] = *(const uint4 *)(p + (c0 < cols ? c0 : 0u));
    }
}

template <int NCH>
__device__ __forceinline__ void unpack_row(const uint4 (&raw)[NCH], uint32_t cols, int lane, float (&v)[NCH][8]) {
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
        float f[8];
        unpack8(raw[u], f);
        const bool ok = slot_col<true>(lane, u, 0) < cols;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[u][i] = ok ? f[i] : 0.f;
    }
}

template <int NCH, bool VEC>
__device__ __forceinline__ void load_row(const uint16_t *__restrict__ p, uint32_t cols, int lane, float (&v)[NCH][8]) {
    if (VEC) {
        uint4 raw[NCH];
        load_raw<NCH>(p, cols, lane, raw);
#pragma unroll
        for (int u = 0; u < NCH; ++u) pin4(raw[u]);   // all chunks issued before the first wait
        unpack_row<NCH>(raw, cols, lane, v);
        return;
    }
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = slot_col<false>(lane, u, i);
            v[u][i] = c < cols ? sh_dev_h2f(p[c]) : 0.f;
        }
}

template <int NCH, bool VEC>
__device__ __forceinline__ void store_row(uint16_t *__restrict__ p, uint32_t cols, int lane, const float (&v)[NCH][8]) {
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
        if (VEC) {
            const uint32_t c0 = slot_col<true>(lane, u, 0);
            if (c0 < cols) *(uint4 *)(p + c0) = pack8(v[u]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t c = slot_col<false>(lane, u, i);
                if (c < cols) p[c] = sh_dev_f2h(v[u][i]);
            }
        }
    }
}

// y = (x - mean) rsqrt(var + eps) gamma + beta per row (biased variance, two-pass over registers).
template <int NCH, bool VEC>
__global__ __launch_bounds__(256) void k_layernorm(uint16_t *y, const uint16_t *x, const uint16_t *gamma, const uint16_t *beta,
                                                   uint32_t rows, uint32_t cols, uint64_t ldy, uint64_t ldx, float eps) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * kRowWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    float v[NCH][8], g[NCH][8], b[NCH][8];
    if (VEC) {                                        // x, gamma and beta loads in flight together
        uint4 rx[NCH], rg[NCH], rb[NCH];
        load_raw<NCH>(x + row * ldx, cols, lane, rx);
        load_raw<NCH>(gamma, cols, lane, rg);
        load_raw<NCH>(beta, cols, lane, rb);
#pragma unroll
        for (int u = 0; u < NCH; ++u) {               // pin all three here: the compiler would otherwise sink
            pin4(rx[u]);                              // the gamma / beta loads past the reductions
            pin4(rg[u]);
            pin4(rb[u]);
        }
        unpack_row<NCH>(rx, cols, lane, v);
        unpack_row<NCH>(rg, cols, lane, g);
        unpack_row<NCH>(rb, cols, lane, b);
    } else {
        load_row<NCH, VEC>(x + row * ldx, cols, lane, v);
        load_row<NCH, VEC>(gamma, cols, lane, g);
        load_row<NCH, VEC>(beta, cols, lane, b);
    }
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) s += v[u][i];
    const float inv_n = 1.f / (float)cols;
    const float mean = sh_wave_sum(s) * inv_n;
    float q = 0.f;
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float d = slot_col<VEC>(lane, u, i) < cols ? v[u][i] - mean : 0.f;
            q += d * d;
        }
    const float rs = sh_fast_rsq(sh_wave_sum(q) * inv_n + eps);
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) v[u][i] = (v[u][i] - mean) * rs * g[u][i] + b[u][i];
    store_row<NCH, VEC>(y + row * ldy, cols, lane, v);
}

// LayerNorm with rows spread over LPR-lane groups (LPR = 32: two rows per wavefront; 64: one), NCH 16-byte
// chunks per lane, each group walking rows row0, row0 + groups, ...: the next row's loads are issued before the
// current row's statistics, so every group keeps two rows in flight; gamma and beta are loaded once per group.
// Same two-pass statistics as k_layernorm (mean, then the mean of squared deviations, fp32).
template <int LPR, int NCH, bool NT>
__global__ __launch_bounds__(256) void k_layernorm_p(uint16_t *y, const uint16_t *x, const uint16_t *gamma, const uint16_t *beta,
                                                     uint32_t rows, uint32_t cols, uint64_t ldy, uint64_t ldx, float eps) {
    constexpr int GPW = 64 / LPR;                         // row groups per wavefront
    const int lane = threadIdx.x & 63, gl = lane % LPR;
    const uint32_t group = (blockIdx.x * 4 + (threadIdx.x >> 6)) * GPW + lane / LPR;
    const uint32_t ngroups = gridDim.x * 4 * GPW;
    auto col = [&](int u) { return 8u * (uint32_t)(gl + LPR * u); };
    float g[NCH][8], b[NCH][8];
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
        const bool ok = col(u) < cols;
        float fg[8], fb[8];
        unpack8(*(const uint4 *)(gamma + (ok ? col(u) : 0u)), fg);
        unpack8(*(const uint4 *)(beta + (ok ? col(u) : 0u)), fb);
#pragma unroll
        for (int i = 0; i < 8; ++i) { g[u][i] = fg[i]; b[u][i] = fb[i]; }
    }
    uint32_t row = group;
    uint4 cur[NCH];
    const uint32_t r0 = row < rows ? row : 0u;
#pragma unroll
    for (int u = 0; u < NCH; ++u) cur[u] = ld16<false>(x + r0 * ldx + (col(u) < cols ? col(u) : 0u));
    const float inv_n = 1.f / (float)cols;
    for (; row < rows; row += ngroups) {                  // the trip count differs between the groups of a wave
        const uint32_t nrow = row + ngroups < rows ? row + ngroups : row;
        uint4 nxt[NCH];
#pragma unroll
        for (int u = 0; u < NCH; ++u) nxt[u] = ld16<false>(x + nrow * ldx + (col(u) < cols ? col(u) : 0u));
        float v[NCH][8];
        float s = 0.f;
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            unpack8(cur[u], v[u]);
            const bool ok = col(u) < cols;
#pragma unroll
            for (int i = 0; i < 8; ++i) { v[u][i] = ok ? v[u][i] : 0.f; s += v[u][i]; }
        }
#pragma unroll
        for (int o = LPR / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        const float mean = s * inv_n;
        float q = 0.f;
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            const bool ok = col(u) < cols;
#pragma unroll
            for (int i = 0; i < 8; ++i) { const float d = ok ? v[u][i] - mean : 0.f; q += d * d; }
        }
#pragma unroll
        for (int o = LPR / 2; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
        const float rs = sh_fast_rsq(q * inv_n + eps);
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            if (col(u) >= cols) continue;
            float o8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) o8[i] = (v[u][i] - mean) * rs * g[u][i] + b[u][i];
            st16(y + row * ldy + col(u), pack8(o8), NT);
        }
#pragma unroll
        for (int u = 0; u < NCH; ++u) cur[u] = nxt[u];
    }
}

// Row statistics of k_layernorm_p's rows (the same two passes in fp32), as (mean, 1 / sqrt(var + eps)) pairs.
template <int LPR, int NCH>
__global__ __launch_bounds__(256) void k_row_stats(float2 *stats, const uint16_t *x, uint32_t rows, uint32_t cols, uint64_t ldx,
                                                   float eps) {
    constexpr int GPW = 64 / LPR;
    const int lane = threadIdx.x & 63, gl = lane % LPR;
    const uint32_t group = (blockIdx.x * 4 + (threadIdx.x >> 6)) * GPW + lane / LPR;
    const uint32_t ngroups = gridDim.x * 4 * GPW;
    auto col = [&](int u) { return 8u * (uint32_t)(gl + LPR * u); };
    const float inv_n = 1.f / (float)cols;
    uint32_t row = group;
    uint4 cur[NCH];
    const uint32_t r0 = row < rows ? row : 0u;
#pragma unroll
    for (int u = 0; u < NCH; ++u) cur[u] = *(const uint4 *)(x + r0 * ldx + (col(u) < cols ? col(u) : 0u));
    for (; row < rows; row += ngroups) {
        const uint32_t nrow = row + ngroups < rows ? row + ngroups : row;
        uint4 nxt[NCH];
#pragma unroll
        for (int u = 0; u < NCH; ++u) nxt[u] = *(const uint4 *)(x + nrow * ldx + (col(u) < cols ? col(u) : 0u));
        float v[NCH][8];
        float s = 0.f;
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            unpack8(cur[u], v[u]);
            const bool ok = col(u) < cols;
#pragma unroll
            for (int i = 0; i < 8; ++i) { v[u][i] = ok ? v[u][i] : 0.f; s += v[u][i]; }
        }
#pragma unroll
        for (int o = LPR / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        const float mean = s * inv_n;
        float q = 0.f;
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            const bool ok = col(u) < cols;
#pragma unroll
            for (int i = 0; i < 8; ++i) { const float d = ok ? v[u][i] - mean : 0.f; q += d * d; }
        }
#pragma unroll
        for (int o = LPR / 2; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
        if (gl == 0) stats[row] = make_float2(mean, sh_fast_rsq(q * inv_n + eps));
#pragma unroll
        for (int u = 0; u < NCH; ++u) cur[u] = nxt[u];
    }
}

// The weight side of a LayerNorm fold, one column n per thread walking k: wp = r16(gamma_k w), c += wp (fp32),
// d += beta_k w (fp32), then d += bias.
__global__ __launch_bounds__(256) void k_ln_fold(uint16_t *wp, float *c, float *d, const uint16_t *w, const uint16_t *gamma,
                                                 const uint16_t *beta, const uint16_t *bias, uint32_t K, uint32_t N,
                                                 uint64_t ldw, uint64_t ldwp) {
    const uint32_t n = blockIdx.x * 256u + threadIdx.x;
    if (n >= N) return;
    float cs = 0.f, ds = 0.f;
    for (uint32_t k = 0; k < K; ++k) {
        const float wv = sh_dev_h2f(w[(uint64_t)k * ldw + n]);
        const uint16_t h = sh_dev_f2h(sh_dev_h2f(gamma[k]) * wv);
        wp[(uint64_t)k * ldwp + n] = h;
        cs += sh_dev_h2f(h);
        ds = fmaf(sh_dev_h2f(beta[k]), wv, ds);
    }
    c[n] = cs;
    d[n] = ds + (bias ? sh_dev_h2f(bias[n]) : 0.f);
}

// Streaming 1-D copy of n16 16-byte chunks: U chunks per thread, all loaded before any is stored, one pass per
// thread (no grid-stride loop: a thread's next loads would queue behind its stores in the memory counter).
template <int U, bool NT>
__global__ __launch_bounds__(256) void k_copy16(uint4 *__restrict__ dst, const uint4 *__restrict__ src, uint64_t n16) {
    const uint64_t base = (uint64_t)blockIdx.x * 256u * U + threadIdx.x;
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint64_t i = base + (uint64_t)u * 256u;
        v[u] = ld16<NT>(src + (i < n16 ? i : 0));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint64_t i = base + (uint64_t)u * 256u;
        if (i < n16) st16(dst + i, v[u], NT);
    }
}

__global__ __launch_bounds__(256) void k_copy1(uint8_t *dst, const uint8_t *src, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256u) dst[i] = src[i];
}

// y = softmax(scale x) per row: exp(scale x - max) = 2^(c x - m), c = scale log2(e), m = max(c x).
template <int NCH, bool VEC>
__global__ __launch_bounds__(256) void k_softmax(uint16_t *y, const uint16_t *x, uint32_t rows, uint32_t cols, uint64_t ld, float c) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * kRowWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    float v[NCH][8];
    load_row<NCH, VEC>(x + row * ld, cols, lane, v);
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[u][i] *= c;
            if (slot_col<VEC>(lane, u, i) < cols) m = fmaxf(m, v[u][i]);
        }
    m = sh_wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float e = slot_col<VEC>(lane, u, i) < cols ? sh_fast_exp2(v[u][i] - m) : 0.f;
            v[u][i] = e;
            s += e;
        }
    const float inv = 1.f / sh_wave_sum(s);
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) v[u][i] *= inv;
    store_row<NCH, VEC>(y + row * ld, cols, lane, v);
}

// Short rows (cols <= 8 LPR, 16-byte aligned): LPR lanes per row, 64 / LPR rows per wavefront and RIT such
// groups per wavefront, every load of the RIT groups issued before the first reduction, so each lane keeps RIT
// 16-byte loads in flight and no lane idles on a row narrower than a wavefront. Same arithmetic as k_softmax.
template <int LPR, int RIT>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
template <int LPR, int RIT>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int LPR, int RIT, bool NT>
__global__ __launch_bounds__(256) void k_softmax_narrow(uint16_t *y, const uint16_t *x, uint32_t rows, uint32_t cols, uint64_t ld, float c) {
    constexpr int RPW = 64 / LPR;                     // rows per wavefront per group
    const int lane = threadIdx.x & 63, sub = lane / LPR, l = lane % LPR;
    const uint32_t row0 = (blockIdx.x * kRowWaves + (threadIdx.x >> 6)) * (uint32_t)(RPW * RIT) + (uint32_t)sub;
    const uint32_t c0 = 8u * (uint32_t)l;
    const bool colok = c0 < cols;
    uint4 raw[RIT];
#pragma unroll
    for (int r = 0; r < RIT; ++r) {                   // rows past the end re-read row 0 and are not stored
        const uint32_t row = row0 + (uint32_t)(r * RPW);
        raw[r] = ld16<NT>(x + (row < rows ? row : 0u) * ld + (colok ? c0 : 0u));
    }
#pragma unroll
    for (int r = 0; r < RIT; ++r) pin4(raw[r]);
#pragma unroll
    for (int r = 0; r < RIT; ++r) {
        float v[8];
        unpack8(raw[r], v);
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[i] *= c;
            if (colok) m = fmaxf(m, v[i]);
        }
        m = group_max<LPR, RIT>(m);
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[i] = colok ? sh_fast_exp2(v[i] - m) : 0.f;
            sum += v[i];
        }
        const float inv = 1.f / group_sum<LPR, RIT>(sum);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] *= inv;
        const uint32_t row = row0 + (uint32_t)(r * RPW);
        if (row < rows && colok) st16(y + row * ld + c0, pack8(v), NT);
    }
}

// Rows wider than the register-resident kernels hold: one 256-thread block per row, three passes over it.
__device__ float block_reduce(float v, bool is_max, float *red) {
    v = is_max ? sh_wave_max(v) : sh_wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
    return r;
}

__global__ __launch_bounds__(256) void k_layernorm_wide(uint16_t *y, const uint16_t *x, const uint16_t *gamma, const uint16_t *beta,
                                                        uint32_t cols, uint64_t ldy, uint64_t ldx, float eps) {
    __shared__ float red[4];
    const uint16_t *xr = x + blockIdx.x * ldx;
    uint16_t *yr = y + blockIdx.x * ldy;
    float s = 0.f;
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) s += sh_dev_h2f(xr[c]);
    const float mean = block_reduce(s, false, red) / (float)cols;
    float q = 0.f;
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) { const float d = sh_dev_h2f(xr[c]) - mean; q += d * d; }
    const float rs = sh_fast_rsq(block_reduce(q, false, red) / (float)cols + eps);
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x)
        yr[c] = sh_dev_f2h((sh_dev_h2f(xr[c]) - mean) * rs * sh_dev_h2f(gamma[c]) + sh_dev_h2f(beta[c]));
}

__global__ __launch_bounds__(256) void k_softmax_wide(uint16_t *y, const uint16_t *x, uint32_t cols, uint64_t ld, float c) {
    __shared__ float red[4];
    const uint16_t *xr = x + blockIdx.x * ld;
    uint16_t *yr = y + blockIdx.x * ld;
    float m = -INFINITY;
    for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) m = fmaxf(m, c * sh_dev_h2f(xr[i]));
    m = block_reduce(m, true, red);
    float s = 0.f;
    for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) s += sh_fast_exp2(c * sh_dev_h2f(xr[i]) - m);
    const float inv = 1.f / block_reduce(s, false, red);
    __syncthreads();   // in place: every read of the row above happens before the first store below
    for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) yr[i] = sh_dev_f2h(sh_fast_exp2(c * sh_dev_h2f(xr[i]) - m) * inv);
}

// Elementwise ops over [rows, cols] with one leading dim; item = a 16-byte chunk (VEC) or one half.
template <int OP>
__device__ __forceinline__ float ew(float a, float b, float s) {
    if (OP == OP_SCALE) return a * s;
    if (OP == OP_SILU_MUL) {   // a b / (1 + 2^t), t = -a log2(e) clamped to [-14, 15] (sh_llm.inc.c:152-167)
        const float t = fminf(fmaxf(-a * 1.4426950408889634f, -14.f), 15.f);
        return a * b * sh_fast_rcp(1.f + sh_fast_exp2(t));
    }
    return a + b;   // OP_ADD, OP_BIAS (rounded once to fp16 by the caller)
}

template <int OP, bool VEC, int U, bool NT>
__global__ __launch_bounds__(256) void k_elementwise(uint16_t *y, const uint16_t *a, const uint16_t *b, uint32_t rows,
                                                     uint32_t per_row, ShDiv div, uint64_t ld, float s, uint32_t items) {
    // U items per thread, issued together
    const uint32_t base = blockIdx.x * (256u * U) + threadIdx.x;
    (void)rows;
    if (VEC) {
        // all loads of the thread's items first (an item past the end reloads item 0 and is not stored), then
        // compute and store: no load waits behind a store even when y aliases a
        uint4 ra[U], rb[U];
        uint64_t off[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t it = base + u * 256u;
            ok[u] = it < items;
            const uint32_t itc = ok[u] ? it : 0u;
            const uint32_t r = sh_div(itc, div), cc = itc - r * per_row;
            off[u] = r * ld + 8ull * cc;
            ra[u] = ld16<NT>(a + off[u]);
            if (OP == OP_ADD || OP == OP_SILU_MUL) rb[u] = ld16<NT>(b + off[u]);
            else if (OP == OP_BIAS) rb[u] = *(const uint4 *)(b + 8ull * cc);
            else rb[u] = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (!ok[u]) continue;
            if (OP == OP_GELU) {                      // on fp16 pairs, as the GEMM epilogue does
                const uint4 q = ra[u];
                st16(y + off[u], make_uint4(sh_gelu_u32(q.x), sh_gelu_u32(q.y), sh_gelu_u32(q.z), sh_gelu_u32(q.w)), NT);
                continue;
            }
            float fa[8], fb[8];
            unpack8(ra[u], fa);
            unpack8(rb[u], fb);
#pragma unroll
            for (int i = 0; i < 8; ++i) fa[i] = ew<OP>(fa[i], fb[i], s);
            st16(y + off[u], pack8(fa), NT);
        }
        return;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t it = base + u * 256u;
        if (it >= items) break;
        const uint32_t r = sh_div(it, div), cc = it - r * per_row;
        const uint64_t off = r * ld + cc;
        float fb = 0.f;
        if (OP == OP_ADD || OP == OP_SILU_MUL) fb = sh_dev_h2f(b[off]);
        else if (OP == OP_BIAS) fb = sh_dev_h2f(b[cc]);
        if (OP == OP_GELU) {
            const uint32_t h = a[off];
            y[off] = (uint16_t)sh_gelu_u32(h | (h << 16));
        } else {
            y[off] = sh_dev_f2h(ew<OP>(sh_dev_h2f(a[off]), fb, s));
        }
    }
}

// dst[cols, rows] = src[rows, cols]^T, 128 x 128 tile per block, 8 x 8 blocks per thread.
template <bool NT>
__global__ __launch_bounds__(256) void k_transpose8(uint16_t *dst, const uint16_t *src, uint32_t rows, uint32_t cols,
                                                    uint64_t lds, uint64_t ldd) {
    __shared__ uint4 tile[128 * 16];                      // [dst row local][16-byte chunk ^ swizzle]
    const int t = threadIdx.x;
    const uint32_t tr = blockIdx.y * 128u, tc = blockIdx.x * 128u;
    const int br = t >> 4, bc = t & 15;
    const uint32_t r0 = tr + 8u * br, c0 = tc + 8u * bc;
    if (r0 < rows && c0 < cols) {                         // rows % 8 == cols % 8 == 0: blocks are whole
        uint32_t w[8][4];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 q = ld16<NT>(src + (uint64_t)(r0 + i) * lds + c0);
            w[i][0] = q.x; w[i][1] = q.y; w[i][2] = q.z; w[i][3] = q.w;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {                     // dst row c0 + j = column j of the block
            uint32_t o[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t lo = w[2 * p][j >> 1], hi = w[2 * p + 1][j >> 1];
                o[p] = (j & 1) ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
            }
            const int R = 8 * bc + j;
            tile[R * 16 + (br ^ ((R >> 3) & 15))] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
    __syncthreads();
    const int C = t & 15;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int R = (t >> 4) + 16 * k;
        const uint32_t drow = tc + R, dcol = tr + 8u * C;
        if (drow < cols && dcol < rows) st16(dst + (uint64_t)drow * ldd + dcol, tile[R * 16 + (C ^ ((R >> 3) & 15))], NT);
    }
}

// Any shape / alignment: 32 x 32 tiles through LDS, one half per access.
__global__ __launch_bounds__(256) void k_transpose1(uint16_t *dst, const uint16_t *src, uint32_t rows, uint32_t cols,
                                                    uint64_t lds, uint64_t ldd) {
    __shared__ uint16_t tile[32][33];
    const uint32_t tr = blockIdx.y * 32u, tc = blockIdx.x * 32u;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int i = ty; i < 32; i += 8) {
        const uint32_t r = tr + i, c = tc + tx;
        if (r < rows && c < cols) tile[i][tx] = src[(uint64_t)r * lds + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const uint32_t dr = tc + i, dc = tr + tx;
        if (dr < cols && dc < rows) dst[(uint64_t)dr * ldd + dc] = tile[tx][i];
    }
}

// ---- host side ---------------------------------------------------------------------------------------
bool vec_ok(uint32_t cols, std::initializer_list<uint64_t> ptrs, std::initializer_list<uint32_t> lds) {
    if (cols % 8) return false;
    for (uint64_t p : ptrs) if (p && !sh_aligned16(p)) return false;
    for (uint32_t l : lds) if (l % 8) return false;
    return true;
}

// Host-side validation; HIP is initialised only once the arguments are known to be usable.
bool check_args(const char *op, uint64_t y, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld) {
    if (rows == 0 || cols == 0) return false;               // nothing to do
    if (!y || !x) { sh_set_error(-1, "[%s] NULL tensor address", op); return false; }
    if (ld < cols) { sh_set_error(-1, "[%s] ld %u < cols %u", op, ld, cols); return false; }
    sh_ensure_init();
    return true;
}

void launch_layernorm(uint64_t y, uint64_t x, uint64_t g, uint64_t b, uint32_t rows, uint32_t cols, uint32_t ldy, uint32_t ldx, float eps) {
    hipStream_t st = sh_stream();
    uint16_t *Y = (uint16_t *)y; const uint16_t *X = (const uint16_t *)x, *G = (const uint16_t *)g, *B = (const uint16_t *)b;
    if (cols > 8192) {
        hipLaunchKernelGGL(k_layernorm_wide, dim3(rows), dim3(256), 0, st, Y, X, G, B, cols, (uint64_t)ldy, (uint64_t)ldx, eps);
        sh_launch_ok("sh_layernorm");
        return;
    }
    const bool vec = vec_ok(cols, {y, x, g, b}, {ldy, ldx});
    if (vec && cols <= 4096) {
        // row groups of 32 lanes up to 1024 columns (two rows per wavefront), else 64; one row per group while
        // that keeps up to 32 blocks per CU, beyond it rows are walked in turn (two in flight per group).
        // [131072 x 768]: 32 blocks per CU 6.0 TB/s, 16 5.8, 64 5.7, one row per group 5.6
        const uint32_t lpr = cols <= 1024 ? 32 : 64, gpb = 4 * (64 / lpr);
        const uint32_t cap = (uint32_t)(sh_num_cus() > 0 ? sh_num_cus() : 256) * 32;
        const dim3 g(std::max<uint32_t>(1, std::min<uint32_t>(sh_cdiv(rows, gpb), cap)));
        const uint32_t nt = (uint64_t)rows * cols * 2 >= kNtBytes;
#define SH_LNP(L, N) do { if (nt) hipLaunchKernelGGL((k_layernorm_p<L, N, true>), g, dim3(256), 0, st, Y, X, G, B, rows, cols, (uint64_t)ldy, (uint64_t)ldx, eps); \
                         else hipLaunchKernelGGL((k_layernorm_p<L, N, false>), g, dim3(256), 0, st, Y, X, G, B, rows, cols, (uint64_t)ldy, (uint64_t)ldx, eps); } while (0)
        if (lpr == 32) { if (cols <= 256) SH_LNP(32, 1); else if (cols <= 512) SH_LNP(32, 2); else if (cols <= 768) SH_LNP(32, 3); else SH_LNP(32, 4); }
        else { if (cols <= 2048) SH_LNP(64, 4); else if (cols <= 3072) SH_LNP(64, 6); else SH_LNP(64, 8); }
#undef SH_LNP
        sh_launch_ok("sh_layernorm");
        return;
    }
    const dim3 grid(sh_cdiv(rows, kRowWaves)), block(256);
#define SH_LN(N) do { if (vec) hipLaunchKernelGGL((k_layernorm<N, true>), grid, block, 0, st, Y, X, G, B, rows, cols, (uint64_t)ldy, (uint64_t)ldx, eps); \
                      else hipLaunchKernelGGL((k_layernorm<N, false>), grid, block, 0, st, Y, X, G, B, rows, cols, (uint64_t)ldy, (uint64_t)ldx, eps); } while (0)
    if (cols <= 512) SH_LN(1); else if (cols <= 1024) SH_LN(2); else if (cols <= 2048) SH_LN(4); else if (cols <= 4096) SH_LN(8); else SH_LN(16);
#undef SH_LN
    sh_launch_ok("sh_layernorm");
}

void launch_elementwise(int op, uint64_t y, uint64_t a, uint64_t b, uint32_t rows, uint32_t cols, uint32_t ld, float s, const char *name) {
    hipStream_t st = sh_stream();
    const bool vec = vec_ok(cols, {y, a, b}, {ld});
    const uint32_t per_row = vec ? cols / 8 : cols;
    const uint64_t items64 = (uint64_t)rows * per_row;
    if (items64 > 0xFFFFFFFFull - 4096) { sh_set_error(-1, "[%s] %u x %u is too large", name, rows, cols); return; }
    const uint32_t items = (uint32_t)items64;
    const ShDiv div = sh_make_div(per_row);
    uint16_t *Y = (uint16_t *)y; const uint16_t *A = (const uint16_t *)a, *B = (const uint16_t *)b;
    const uint32_t nt = (uint64_t)rows * cols * 2 >= kNtBytes;
    // one item per thread (the most workgroups in flight) for GELU, whose VALU work wants the most wavefronts, and
    // for streamed (nontemporal) outputs; four per thread for the other ops below it (fewer, fuller launches).
    // Measured on [131072 x 3072] GELU: 6.2 against 5.7 TB/s; at the configured sizes add / add_bias prefer four.
    const bool one = op == OP_GELU || nt;
    const dim3 grid(sh_cdiv(items, 256u * (one ? 1u : 4u))), block(256);
#define SH_EW(OP) do { \
        if (one) { if (vec && nt) hipLaunchKernelGGL((k_elementwise<OP, true, 1, true>), grid, block, 0, st, Y, A, B, rows, per_row, div, (uint64_t)ld, s, items); \
                   else if (vec) hipLaunchKernelGGL((k_elementwise<OP, true, 1, false>), grid, block, 0, st, Y, A, B, rows, per_row, div, (uint64_t)ld, s, items); \
                   else hipLaunchKernelGGL((k_elementwise<OP, false, 1, false>), grid, block, 0, st, Y, A, B, rows, per_row, div, (uint64_t)ld, s, items); } \
        else { if (vec) hipLaunchKernelGGL((k_elementwise<OP, true, 4, false>), grid, block, 0, st, Y, A, B, rows, per_row, div, (uint64_t)ld, s, items); \
               else hipLaunchKernelGGL((k_elementwise<OP, false, 4, false>), grid, block, 0, st, Y, A, B, rows, per_row, div, (uint64_t)ld, s, items); } } while (0)
    switch (op) {
        case OP_GELU: SH_EW(OP_GELU); break;
        case OP_ADD: SH_EW(OP_ADD); break;
        case OP_BIAS: SH_EW(OP_BIAS); break;
        case OP_SILU_MUL: SH_EW(OP_SILU_MUL); break;
        default: SH_EW(OP_SCALE); break;
    }
#undef SH_EW
    sh_launch_ok(name);
}


// ---- Llama-style decoder row ops (reference runtime/sh_llm.inc.c) ------------------------------------------
constexpr uint32_t kLlmPad = 0xFFFFu;      // SH_LLM_PAD
__device__ __forceinline__ uint32_t comp4r(const uint4 &q, int i) { return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w; }

// y = x rsqrt(mean(x^2) + eps) gamma per row, fp32 statistics (sh_llm.inc.c:91-120). Same layout as k_layernorm.
template <int NCH, bool VEC>
__global__ __launch_bounds__(256) void k_rmsnorm(uint16_t *y, const uint16_t *x, const uint16_t *gamma, uint32_t rows,
                                                 uint32_t cols, uint64_t ld, float eps) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * kRowWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    float v[NCH][8], g[NCH][8];
    if (VEC) {
        uint4 rx[NCH], rg[NCH];
        load_raw<NCH>(x + row * ld, cols, lane, rx);
        load_raw<NCH>(gamma, cols, lane, rg);
#pragma unroll
        for (int u = 0; u < NCH; ++u) { pin4(rx[u]); pin4(rg[u]); }
        unpack_row<NCH>(rx, cols, lane, v);
        unpack_row<NCH>(rg, cols, lane, g);
    } else {
        load_row<NCH, VEC>(x + row * ld, cols, lane, v);
        load_row<NCH, VEC>(gamma, cols, lane, g);
    }
    float q = 0.f;
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) q += v[u][i] * v[u][i];
    const float rs = sh_fast_rsq(sh_wave_sum(q) / (float)cols + eps);
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) v[u][i] = v[u][i] * rs * g[u][i];
    store_row<NCH, VEC>(y + row * ld, cols, lane, v);
}

// softmax(scale x) per row over the keys j with tok_k[j] <= tok_q[row] (unsigned); a padding query row, or one
// with no allowed key, is uniform 1/cols (sh_llm.inc.c:175-248; run.py:186-196). c = scale log2(e) > 0.
template <int NCH, bool VEC>
__global__ __launch_bounds__(256) void k_softmax_masked(uint16_t *y, const uint16_t *x, uint32_t rows, uint32_t cols, uint64_t ld,
                                                        float c, const uint16_t *tok_q, const uint16_t *tok_k) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * kRowWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t ti = tok_q[row];
    float v[NCH][8];
    bool keep[NCH][8];
    load_row<NCH, VEC>(x + row * ld, cols, lane, v);
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
        if (VEC) {
            const uint32_t c0 = slot_col<true>(lane, u, 0);
            const uint4 t = *(const uint4 *)(tok_k + (c0 < cols ? c0 : 0u));
#pragma unroll
            for (int i = 0; i < 8; ++i)
                keep[u][i] = c0 + i < cols && ((comp4r(t, i >> 1) >> (16 * (i & 1))) & 0xFFFFu) <= ti;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t col = slot_col<false>(lane, u, i);
                keep[u][i] = col < cols && (uint32_t)tok_k[col] <= ti;
            }
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[u][i] *= c;
            if (keep[u][i]) m = fmaxf(m, v[u][i]);
        }
    m = sh_wave_max(m);
    const bool uni = ti == kLlmPad || m == -INFINITY;
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float e = uni ? 1.f : (keep[u][i] ? sh_fast_exp2(v[u][i] - m) : 0.f);
            v[u][i] = e;
            if (slot_col<VEC>(lane, u, i) < cols) s += e;
        }
    const float inv = 1.f / sh_wave_sum(s);
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) v[u][i] *= inv;
    store_row<NCH, VEC>(y + row * ld, cols, lane, v);
}

// Rotate-half RoPE (sh_llm.inc.c:127-150): item = (row, p), p < cols / 2 -> head p / half, pair j = p % half:
// y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin with x1 = x[h dh + j], x2 = x[h dh + half + j], the row's table
// entry cos = t[j], sin = t[half + j]. In place allowed (each item reads and writes its own pair).
__global__ __launch_bounds__(256) void k_rope(uint16_t *y, const uint16_t *x, const uint16_t *tab, uint64_t ld, uint64_t ldt,
                                              uint32_t half, ShDiv per_row, ShDiv by_half, uint32_t items) {
    const uint32_t it = blockIdx.x * 256u + threadIdx.x;
    if (it >= items) return;
    const uint32_t row = sh_div(it, per_row), p = it - row * per_row.d;
    const uint32_t h = sh_div(p, by_half), j = p - h * half;
    const uint64_t o1 = (uint64_t)row * ld + 2ull * h * half + j, o2 = o1 + half;
    const float x1 = sh_dev_h2f(x[o1]), x2 = sh_dev_h2f(x[o2]);
    const float cs = sh_dev_h2f(tab[(uint64_t)row * ldt + j]), sn = sh_dev_h2f(tab[(uint64_t)row * ldt + half + j]);
    y[o1] = sh_dev_f2h(x1 * cs - x2 * sn);
    y[o2] = sh_dev_f2h(x2 * cs + x1 * sn);
}

// SmolVLM connector pixel shuffle (sh_llm.inc.c:344-362): dst token t = (gr, gb) of the (grid/s)^2 output tokens
// is s chunks of s D elements: chunk i = src rows (gr s + i) grid + gb s .. + s (contiguous). 16-byte items.
__global__ __launch_bounds__(256) void k_pixel_shuffle(uint4 *dst, const uint4 *src, uint32_t grid, uint32_t s, uint32_t dv,
                                                       uint32_t g, uint32_t items) {
    const uint32_t it = blockIdx.x * 256u + threadIdx.x;   // dst item (16 bytes); dv = D / 8 items per patch
    if (it >= items) return;
    const uint32_t chunk = s * dv, per_tok = s * chunk, t = it / per_tok, r = it - t * per_tok, i = r / chunk, e = r - i * chunk;
    const uint32_t gr = t / g, gb = t - gr * g;
    dst[it] = src[(uint64_t)((gr * s + i) * grid + gb * s) * dv + e];
}

__global__ __launch_bounds__(256) void k_pixel_shuffle1(uint16_t *dst, const uint16_t *src, uint32_t grid, uint32_t s, uint32_t D,
                                                        uint32_t g, uint32_t items) {
    const uint32_t it = blockIdx.x * 256u + threadIdx.x;   // dst element
    if (it >= items) return;
    const uint32_t chunk = s * D, per_tok = s * chunk, t = it / per_tok, r = it - t * per_tok, i = r / chunk, e = r - i * chunk;
    const uint32_t gr = t / g, gb = t - gr * g;
    dst[it] = src[(uint64_t)((gr * s + i) * grid + gb * s) * D + e];
}
}  // namespace

// One load of every 64-byte line of [base, base + 64 lines): the lines come into L2 and the Infinity Cache for the
// kernels that read them next, and nothing is written (the empty asm keeps each load, and the wave waits for it).
__global__ __launch_bounds__(256) void k_prefetch(const uint8_t *__restrict__ base, uint64_t lines) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < lines; i += (uint64_t)gridDim.x * 256u) {
        const uint32_t v = *(const uint32_t *)(base + i * 64);
        asm volatile("" ::"v"(v));
    }
}

extern "C" {

void sh_layernorm(uint64_t y, uint64_t x, uint64_t gamma, uint64_t beta, uint32_t rows, uint32_t cols, uint32_t ld, float eps, uint32_t) {
    if (!check_args("sh_layernorm", y, x, rows, cols, ld)) return;
    if (!gamma || !beta) { sh_set_error(-1, "[sh_layernorm] NULL gamma/beta"); return; }
    launch_layernorm(y, x, gamma, beta, rows, cols, ld, ld, eps);
}

void sh_layernorm_ld(uint64_t y, uint64_t x, uint64_t gamma, uint64_t beta, uint32_t rows, uint32_t cols, uint32_t ldy, uint32_t ldx, float eps) {
    if (!check_args("sh_layernorm_ld", y, x, rows, cols, ldy < ldx ? ldy : ldx)) return;
    if (!gamma || !beta) { sh_set_error(-1, "[sh_layernorm_ld] NULL gamma/beta"); return; }
    launch_layernorm(y, x, gamma, beta, rows, cols, ldy, ldx, eps);
}

void sh_row_stats(uint64_t stats, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, float eps) {
    if (!check_args("sh_row_stats", stats, x, rows, cols, ld)) return;
    if (stats % 8) { sh_set_error(-1, "[sh_row_stats] stats must be 8-byte aligned"); return; }
    if (!vec_ok(cols, {x}, {ld}) || cols > 4096) {
        sh_set_error(-1, "[sh_row_stats] needs 16-byte aligned rows (cols, ld %% 8 == 0) of at most 4096 columns");
        return;
    }
    hipStream_t st = sh_stream();
    const uint32_t lpr = cols <= 1024 ? 32 : 64, gpb = 4 * (64 / lpr);
    const uint32_t cap = (uint32_t)(sh_num_cus() > 0 ? sh_num_cus() : 256) * 16;
    const dim3 g(std::max<uint32_t>(1, std::min<uint32_t>(sh_cdiv(rows, gpb), cap)));
    float2 *S = (float2 *)stats; const uint16_t *X = (const uint16_t *)x;
#define SH_RS(L, N) hipLaunchKernelGGL((k_row_stats<L, N>), g, dim3(256), 0, st, S, X, rows, cols, (uint64_t)ld, eps)
    if (lpr == 32) { if (cols <= 256) SH_RS(32, 1); else if (cols <= 512) SH_RS(32, 2); else if (cols <= 768) SH_RS(32, 3); else SH_RS(32, 4); }
    else { if (cols <= 2048) SH_RS(64, 4); else if (cols <= 3072) SH_RS(64, 6); else SH_RS(64, 8); }
#undef SH_RS
    sh_launch_ok("sh_row_stats");
}

void sh_ln_fold(uint64_t wp, uint64_t c, uint64_t d, uint64_t w, uint64_t gamma, uint64_t beta, uint64_t bias,
                uint32_t K, uint32_t N, uint32_t ldw, uint32_t ldwp) {
    if (K == 0 || N == 0) return;
    if (!wp || !c || !d || !w || !gamma || !beta) { sh_set_error(-1, "[sh_ln_fold] NULL address"); return; }
    if (ldw < N || ldwp < N) { sh_set_error(-1, "[sh_ln_fold] ldw %u / ldwp %u < N %u", ldw, ldwp, N); return; }
    sh_ensure_init();
    hipLaunchKernelGGL(k_ln_fold, dim3(sh_cdiv(N, 256)), dim3(256), 0, sh_stream(), (uint16_t *)wp, (float *)c, (float *)d,
                       (const uint16_t *)w, (const uint16_t *)gamma, (const uint16_t *)beta, (const uint16_t *)bias, K, N,
                       (uint64_t)ldw, (uint64_t)ldwp);
    sh_launch_ok("sh_ln_fold");
}

// HBM -> HBM 1-D copy of `bytes` (reference sh_l1.inc.c:58-61, an iDMA 1-D transfer), stream-ordered on the
// library stream. 16-byte-aligned ends take the streaming chunk kernel; anything else a byte loop.
void sh_dma_copy(uint64_t dst, uint64_t src, uint32_t bytes) {
    if (bytes == 0) return;
    if (!dst || !src) { sh_set_error(-1, "[sh_dma_copy] NULL address"); return; }
    sh_ensure_init();
    hipStream_t st = sh_stream();
    const uint32_t cap = (uint32_t)(sh_num_cus() > 0 ? sh_num_cus() : 256) * 8;
    if ((dst | src | bytes) % 16 == 0) {
        // for streamed sizes one chunk per thread streams best (a 1 GiB copy: 6.2 TB/s against 5.4 with eight);
        // below them eight per thread
        const uint64_t n16 = bytes / 16;
        const bool big = bytes >= kNtBytes;
        const uint32_t per_block = big ? 256u : 256u * 8u;
        const uint32_t blocks = (uint32_t)((n16 + per_block - 1) / per_block);
        if (big) hipLaunchKernelGGL((k_copy16<1, true>), dim3(blocks), dim3(256), 0, st, (uint4 *)dst, (const uint4 *)src, n16);
        else hipLaunchKernelGGL((k_copy16<8, false>), dim3(blocks), dim3(256), 0, st, (uint4 *)dst, (const uint4 *)src, n16);
    } else {
        const uint32_t blocks = (uint32_t)std::min<uint64_t>((bytes + 255) / 256, cap);
        hipLaunchKernelGGL(k_copy1, dim3(blocks), dim3(256), 0, st, (uint8_t *)dst, (const uint8_t *)src, (uint64_t)bytes);
    }
    sh_launch_ok("sh_dma_copy");
}

int sh_prefetch(uint64_t addr, uint64_t bytes) {
    if (bytes == 0) return 0;
    if (!addr) { sh_set_error(-1, "[sh_prefetch] NULL address"); return -1; }
    sh_ensure_init();
    // whole 64-byte lines: the first and last may reach outside the range, but never outside its pages
    const uint64_t base = addr & ~uint64_t(63), lines = (addr + bytes - base + 63) / 64;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((lines + 255) / 256, 8192);
    hipLaunchKernelGGL(k_prefetch, dim3(blocks), dim3(256), 0, sh_stream(), (const uint8_t *)base, lines);
    return sh_launch_ok("sh_prefetch") ? 0 : SH_EHIP;
}

void sh_softmax_rows(uint64_t y, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, float scale, uint32_t) {
    if (!check_args("sh_softmax_rows", y, x, rows, cols, ld)) return;
    hipStream_t st = sh_stream();
    const float c = scale * 1.4426950408889634f;
    uint16_t *Y = (uint16_t *)y; const uint16_t *X = (const uint16_t *)x;
    if (cols > 8192) {
        hipLaunchKernelGGL(k_softmax_wide, dim3(rows), dim3(256), 0, st, Y, X, cols, (uint64_t)ld, c);
        sh_launch_ok("sh_softmax_rows");
        return;
    }
    const bool vec = vec_ok(cols, {y, x}, {ld});
    if (vec && cols <= 256) {
        constexpr int RIT = 4;
        const uint32_t lpr = cols <= 64 ? 8 : cols <= 128 ? 16 : 32;
        const dim3 g(sh_cdiv(rows, kRowWaves * (64 / lpr) * RIT));
        const uint32_t nt = (uint64_t)rows * cols * 2 >= kNtBytes;
        if (lpr == 8) { if (nt) hipLaunchKernelGGL((k_softmax_narrow<8, RIT, true>), g, dim3(256), 0, st, Y, X, rows, cols, (uint64_t)ld, c); else hipLaunchKernelGGL((k_softmax_narrow<8, RIT, false>), g, dim3(256), 0, st, Y, X, rows, cols, (uint64_t)ld, c); }
        else if (lpr == 16) { if (nt) hipLaunchKernelGGL((k_softmax_narrow<16, RIT, true>), g, dim3(256), 0, st, Y, X, rows, cols, (uint64_t)ld, c); else hipLaunchKernelGGL((k_softmax_narrow<16, RIT, false>), g, dim3(256), 0, st, Y, X, rows, cols, (uint64_t)ld, c); }
        else { if (nt) hipLaunchKernelGGL((k_softmax_narrow<32, RIT, true>), g, dim3(256), 0, st, Y, X, rows, cols, (uint64_t)ld, c); else hipLaunchKernelGGL((k_softmax_narrow<32, RIT, false>), g, dim3(256), 0, st, Y, X, rows, cols, (uint64_t)ld, c); }
        sh_launch_ok("sh_softmax_rows");
        return;
    }
    const dim3 grid(sh_cdiv(rows, kRowWaves)), block(256);
#define SH_SM(N) do { if (vec) hipLaunchKernelGGL((k_softmax<N, true>), grid, block, 0, st, Y, X, rows, cols, (uint64_t)ld, c); \
                      else hipLaunchKernelGGL((k_softmax<N, false>), grid, block, 0, st, Y, X, rows, cols, (uint64_t)ld, c); } while (0)
    if (cols <= 512) SH_SM(1); else if (cols <= 1024) SH_SM(2); else if (cols <= 2048) SH_SM(4); else if (cols <= 4096) SH_SM(8); else SH_SM(16);
#undef SH_SM
    sh_launch_ok("sh_softmax_rows");
}

void sh_gelu(uint64_t y, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t) {
    if (!check_args("sh_gelu", y, x, rows, cols, ld)) return;
    launch_elementwise(OP_GELU, y, x, 0, rows, cols, ld, 0.f, "sh_gelu");
}

void sh_add(uint64_t y, uint64_t a, uint64_t b, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t) {
    if (!check_args("sh_add", y, a, rows, cols, ld)) return;
    if (!b) { sh_set_error(-1, "[sh_add] NULL operand"); return; }
    launch_elementwise(OP_ADD, y, a, b, rows, cols, ld, 0.f, "sh_add");
}

void sh_add_bias(uint64_t y, uint64_t x, uint64_t bias_row, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t) {
    if (!check_args("sh_add_bias", y, x, rows, cols, ld)) return;
    if (!bias_row) { sh_set_error(-1, "[sh_add_bias] NULL bias row"); return; }
    launch_elementwise(OP_BIAS, y, x, bias_row, rows, cols, ld, 0.f, "sh_add_bias");
}

void sh_scale(uint64_t y, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, float s, uint32_t) {
    if (!check_args("sh_scale", y, x, rows, cols, ld)) return;
    launch_elementwise(OP_SCALE, y, x, 0, rows, cols, ld, s, "sh_scale");
}

void sh_transpose(uint64_t dst, uint64_t src, uint32_t rows, uint32_t cols, uint32_t ld_src, uint32_t ld_dst, uint32_t) {
    if (!check_args("sh_transpose", dst, src, rows, cols, ld_src)) return;
    if (ld_dst < rows) { sh_set_error(-1, "[sh_transpose] ld_dst %u < rows %u", ld_dst, rows); return; }
    hipStream_t st = sh_stream();
    uint16_t *D = (uint16_t *)dst; const uint16_t *S = (const uint16_t *)src;
    const bool vec = rows % 8 == 0 && vec_ok(cols, {dst, src}, {ld_src, ld_dst});
    if (vec) {
        const dim3 grid(sh_cdiv(cols, 128), sh_cdiv(rows, 128));
        if ((uint64_t)rows * cols * 2 >= kNtBytes)
            hipLaunchKernelGGL((k_transpose8<true>), grid, dim3(256), 0, st, D, S, rows, cols, (uint64_t)ld_src, (uint64_t)ld_dst);
        else
            hipLaunchKernelGGL((k_transpose8<false>), grid, dim3(256), 0, st, D, S, rows, cols, (uint64_t)ld_src, (uint64_t)ld_dst);
    } else {
        const dim3 grid(sh_cdiv(cols, 32), sh_cdiv(rows, 32));
        hipLaunchKernelGGL(k_transpose1, grid, dim3(256), 0, st, D, S, rows, cols, (uint64_t)ld_src, (uint64_t)ld_dst);
    }
    sh_launch_ok("sh_transpose");
}


// ---- Llama-style decoder ops (sh_ops.h:277-307; reference runtime/sh_llm.inc.c) ------------------------------
void sh_rmsnorm(uint64_t y, uint64_t x, uint64_t gamma, uint32_t rows, uint32_t cols, uint32_t ld, float eps, uint32_t) {
    if (cols & 3) { sh_set_error(-1, "[sh_rmsnorm] cols %u %% 4 != 0", cols); return; }            // sh_llm.inc.c:122
    if (cols > 8192) { sh_set_error(-1, "[sh_rmsnorm] cols %u > 8192", cols); return; }
    if (!gamma && rows && cols) { sh_set_error(-1, "[sh_rmsnorm] NULL gamma"); return; }
    if (!check_args("sh_rmsnorm", y, x, rows, cols, ld)) return;
    hipStream_t st = sh_stream();
    const dim3 grid(sh_cdiv(rows, kRowWaves)), block(256);
    const bool vec = vec_ok(cols, {y, x, gamma}, {ld});
    uint16_t *Y = (uint16_t *)y; const uint16_t *X = (const uint16_t *)x, *G = (const uint16_t *)gamma;
#define SH_RMS(N) do { if (vec) hipLaunchKernelGGL((k_rmsnorm<N, true>), grid, block, 0, st, Y, X, G, rows, cols, (uint64_t)ld, eps); \
                       else hipLaunchKernelGGL((k_rmsnorm<N, false>), grid, block, 0, st, Y, X, G, rows, cols, (uint64_t)ld, eps); } while (0)
    if (cols <= 512) SH_RMS(1); else if (cols <= 1024) SH_RMS(2); else if (cols <= 2048) SH_RMS(4); else if (cols <= 4096) SH_RMS(8); else SH_RMS(16);
#undef SH_RMS
    sh_launch_ok("sh_rmsnorm");
}

void sh_rope(uint64_t y, uint64_t x, uint64_t cos_sin, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t ld_table, uint32_t dh, uint32_t) {
    if (dh == 0 || (dh & 7) || cols % dh) {                                                       // sh_llm.inc.c:147
        sh_set_error(-1, "[sh_rope] need dh %% 8 == 0 and cols %% dh == 0 (dh=%u cols=%u)", dh, cols);
        return;
    }
    if (!cos_sin && rows && cols) { sh_set_error(-1, "[sh_rope] NULL table"); return; }
    if (ld_table < dh && rows > 1) { sh_set_error(-1, "[sh_rope] ld_table %u < dh %u", ld_table, dh); return; }
    if (!check_args("sh_rope", y, x, rows, cols, ld)) return;
    const uint64_t items64 = (uint64_t)rows * (cols / 2);
    if (items64 > 0xFFFFFF00ull) { sh_set_error(-1, "[sh_rope] %u x %u is too large", rows, cols); return; }
    const uint32_t items = (uint32_t)items64;
    hipLaunchKernelGGL(k_rope, dim3(sh_cdiv(items, 256u)), dim3(256), 0, sh_stream(), (uint16_t *)y, (const uint16_t *)x,
                       (const uint16_t *)cos_sin, (uint64_t)ld, (uint64_t)ld_table, dh / 2, sh_make_div(cols / 2), sh_make_div(dh / 2), items);
    sh_launch_ok("sh_rope");
}

void sh_silu_mul(uint64_t y, uint64_t a, uint64_t b, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t) {
    if (cols & 3) { sh_set_error(-1, "[sh_silu_mul] cols %u %% 4 != 0", cols); return; }           // sh_llm.inc.c:170
    if (!b && rows && cols) { sh_set_error(-1, "[sh_silu_mul] NULL tensor address"); return; }
    if (!check_args("sh_silu_mul", y, a, rows, cols, ld)) return;
    launch_elementwise(OP_SILU_MUL, y, a, b, rows, cols, ld, 0.f, "sh_silu_mul");
}

void sh_softmax_masked(uint64_t y, uint64_t x, uint32_t rows, uint32_t cols, uint32_t ld, float scale, uint64_t tok_q,
                       uint64_t tok_k, uint32_t) {
    if ((cols & 3) || !(scale > 0.f)) {                                                            // sh_llm.inc.c:244
        sh_set_error(-1, "[sh_softmax_masked] need cols %% 4 == 0 and scale > 0");
        return;
    }
    if (cols > 8192) { sh_set_error(-1, "[sh_softmax_masked] cols %u > 8192", cols); return; }
    if ((!tok_q || !tok_k) && rows && cols) { sh_set_error(-1, "[sh_softmax_masked] NULL token array"); return; }
    if (!check_args("sh_softmax_masked", y, x, rows, cols, ld)) return;
    hipStream_t st = sh_stream();
    const float c = scale * 1.4426950408889634f;
    const dim3 grid(sh_cdiv(rows, kRowWaves)), block(256);
    const bool vec = vec_ok(cols, {y, x, tok_k}, {ld});
    uint16_t *Y = (uint16_t *)y; const uint16_t *X = (const uint16_t *)x, *TQ = (const uint16_t *)tok_q, *TK = (const uint16_t *)tok_k;
#define SH_SMM(N) do { if (vec) hipLaunchKernelGGL((k_softmax_masked<N, true>), grid, block, 0, st, Y, X, rows, cols, (uint64_t)ld, c, TQ, TK); \
                       else hipLaunchKernelGGL((k_softmax_masked<N, false>), grid, block, 0, st, Y, X, rows, cols, (uint64_t)ld, c, TQ, TK); } while (0)
    if (cols <= 512) SH_SMM(1); else if (cols <= 1024) SH_SMM(2); else if (cols <= 2048) SH_SMM(4); else if (cols <= 4096) SH_SMM(8); else SH_SMM(16);
#undef SH_SMM
    sh_launch_ok("sh_softmax_masked");
}

void sh_pixel_shuffle(uint64_t dst, uint64_t src, uint32_t grid, uint32_t D, uint32_t s, uint32_t) {
    if (s == 0 || grid % s) { sh_set_error(-1, "[sh_pixel_shuffle] grid %u not divisible by s %u", grid, s); return; }
    if (grid == 0 || D == 0) return;
    if (!dst || !src) { sh_set_error(-1, "[sh_pixel_shuffle] NULL tensor address"); return; }
    const uint64_t total = (uint64_t)grid * grid * D;
    if (total > 0xFFFFFF00ull) { sh_set_error(-1, "[sh_pixel_shuffle] %u^2 x %u is too large", grid, D); return; }
    sh_ensure_init();
    const uint32_t g = grid / s;
    hipStream_t st = sh_stream();
    if (D % 8 == 0 && sh_aligned16(dst) && sh_aligned16(src)) {
        const uint32_t items = (uint32_t)(total / 8);
        hipLaunchKernelGGL(k_pixel_shuffle, dim3(sh_cdiv(items, 256u)), dim3(256), 0, st, (uint4 *)dst, (const uint4 *)src, grid, s, D / 8, g, items);
    } else {
        hipLaunchKernelGGL(k_pixel_shuffle1, dim3(sh_cdiv((uint32_t)total, 256u)), dim3(256), 0, st, (uint16_t *)dst, (const uint16_t *)src,
                           grid, s, D, g, (uint32_t)total);
    }
    sh_launch_ok("sh_pixel_shuffle");
}

}  // extern "C"
