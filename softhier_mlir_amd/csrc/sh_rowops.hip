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
enum { OP_GELU = 0, OP_ADD = 1, OP_BIAS = 2, OP_SCALE = 3 };

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
    return a + b;   // OP_ADD, OP_BIAS (rounded once to fp16 by the caller)
}

template <int OP, bool VEC>
__global__ __launch_bounds__(256) void k_elementwise(uint16_t *y, const uint16_t *a, const uint16_t *b, uint32_t rows,
                                                     uint32_t per_row, ShDiv div, uint64_t ld, float s, uint32_t items) {
    constexpr int U = 4;   // items per thread, issued together
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
            ra[u] = *(const uint4 *)(a + off[u]);
            if (OP == OP_ADD) rb[u] = *(const uint4 *)(b + off[u]);
            else if (OP == OP_BIAS) rb[u] = *(const uint4 *)(b + 8ull * cc);
            else rb[u] = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (!ok[u]) continue;
            if (OP == OP_GELU) {                      // on fp16 pairs, as the GEMM epilogue does
                const uint4 q = ra[u];
                *(uint4 *)(y + off[u]) = make_uint4(sh_gelu_u32(q.x), sh_gelu_u32(q.y), sh_gelu_u32(q.z), sh_gelu_u32(q.w));
                continue;
            }
            float fa[8], fb[8];
            unpack8(ra[u], fa);
            unpack8(rb[u], fb);
#pragma unroll
            for (int i = 0; i < 8; ++i) fa[i] = ew<OP>(fa[i], fb[i], s);
            *(uint4 *)(y + off[u]) = pack8(fa);
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
        if (OP == OP_ADD) fb = sh_dev_h2f(b[off]);
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
            const uint4 q = *(const uint4 *)(src + (uint64_t)(r0 + i) * lds + c0);
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
        if (drow < cols && dcol < rows) *(uint4 *)(dst + (uint64_t)drow * ldd + dcol) = tile[R * 16 + (C ^ ((R >> 3) & 15))];
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
    const dim3 grid(sh_cdiv(rows, kRowWaves)), block(256);
    const bool vec = vec_ok(cols, {y, x, g, b}, {ldy, ldx});
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
    const dim3 grid(sh_cdiv(items, 256u * 4u)), block(256);
    uint16_t *Y = (uint16_t *)y; const uint16_t *A = (const uint16_t *)a, *B = (const uint16_t *)b;
#define SH_EW(OP) do { if (vec) hipLaunchKernelGGL((k_elementwise<OP, true>), grid, block, 0, st, Y, A, B, rows, per_row, div, (uint64_t)ld, s, items); \
                       else hipLaunchKernelGGL((k_elementwise<OP, false>), grid, block, 0, st, Y, A, B, rows, per_row, div, (uint64_t)ld, s, items); } while (0)
    switch (op) {
        case OP_GELU: SH_EW(OP_GELU); break;
        case OP_ADD: SH_EW(OP_ADD); break;
        case OP_BIAS: SH_EW(OP_BIAS); break;
        default: SH_EW(OP_SCALE); break;
    }
#undef SH_EW
    sh_launch_ok(name);
}

}  // namespace

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
    const dim3 grid(sh_cdiv(rows, kRowWaves)), block(256);
    const bool vec = vec_ok(cols, {y, x}, {ld});
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
        hipLaunchKernelGGL(k_transpose8, grid, dim3(256), 0, st, D, S, rows, cols, (uint64_t)ld_src, (uint64_t)ld_dst);
    } else {
        const dim3 grid(sh_cdiv(cols, 32), sh_cdiv(rows, 32));
        hipLaunchKernelGGL(k_transpose1, grid, dim3(256), 0, st, D, S, rows, cols, (uint64_t)ld_src, (uint64_t)ld_dst);
    }
    sh_launch_ok("sh_transpose");
}

}  // extern "C"
