// sh_gemm family on gfx950 MFMA (reference runtime/sh_gemm.inc.c:12-189, call sites emit_c.py:327-342).
//
// Z[M,N] (+)= X[M,K] . W[K,N], fp16 row-major operands with leading dims, fp32 accumulation, fp16 result.
//
// Kernel: a 256-thread workgroup (2 x 2 wavefronts) computes a BM x BN tile; each wavefront owns a
// (BM/2) x (BN/2) sub-tile as (BM/64) x (BN/64) accumulators of v_mfma_f32_32x32x16_f16. K advances in
// BK = 64 slices through two LDS stages: the next slice is loaded from HBM into registers while the MFMAs
// consume the current stage, then written to the other stage (one barrier per slice).
//  - LDS rows are 64 halves (128 B) = 8 chunks of 16 B; chunk c of row r is stored at c ^ f(r),
//    f(r) = (r ^ (r >> 3)) & 7, which keeps the 16-byte MFMA operand reads of 16 consecutive rows on
//    distinct banks (for 32- and 64-bank LDS alike).
//  - X slices are copied as-is (rows = m, k contiguous). W slices arrive k-major (n contiguous), but the
//    MFMA B operand wants 8 consecutive k per lane, so each thread loads an 8 x 8 block of W and transposes
//    it in registers before the LDS store; LDS then holds W^T rows (n, k contiguous).
//  - The MFMA k order is permuted consistently for both operands: in k-substep s, lane group g = lane/32
//    supplies chunk 4g + s of its row, so all 64 k of a slice are covered once per operand pair.
//  - Epilogue: accumulators (+ z_old, + bias, GELU) are rounded to fp16 into an LDS copy of the tile, then
//    written as 16-byte row chunks (+ residual, rounded again). Split-K writes fp32 partial tiles instead,
//    which a reduction kernel sums in split order (deterministic) and finishes with the same epilogue.
// Workgroup -> tile order is XCD-aware: dispatch deals workgroups round-robin over the XCDs, so workgroup b
// takes logical tile (b % X) * (tiles / X) + b / X and each XCD walks a contiguous run of row-major tiles
// (shared X row panels stay in that XCD's L2).
#include "sh_common.h"
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>
#include <map>
#include <tuple>

namespace {

constexpr int BK = 64;

struct GemmArgs {
    const uint16_t *x, *w;
    uint16_t *z;
    float *part;                 // split-K partials [splits][M][N] (fp32), or null
    const void *bias;            // null, fp16 or fp32 row of N
    const uint16_t *res;         // null or fp16 [M, ldr]
    uint64_t ldx, ldw, ldz, ldr;
    uint32_t M, N, K;
    uint32_t kps;                // K per split (multiple of BK)
    uint32_t tiles_m, tiles_n, splits;
    uint32_t accumulate, bias_fp32, act;
    uint32_t xcd_groups;         // > 1: XCD-aware block remap with this many XCDs (requires divisibility)
    uint32_t group_m;            // > 1: tiles ordered in bands of this many tile rows, column by column within a band
    const float *ln_stats;       // LayerNorm fold (or null): (mu, r) per row, fp32 [M][2], or ln_parts partials ...
    const float *ln_c;           // ... and c per column (fp32 [N]); the fp32 bias row is then d
    uint32_t ln_parts;           // > 0: ln_stats holds ln_parts (sum, M2) pairs of 32 columns per row (row_partials)
    float ln_eps;                // ... and the statistics are formed with this eps
    float *stats_out;            // or null: the (sum, M2) pairs of every 32 columns of each stored row, [M][N / 32]
};

// (mu, r = 1 / sqrt(var + eps)) of row gm for the LayerNorm fold: given (ln_parts == 0), or formed from the row's
// ln_parts partials (s_b, M2_b) of 32 columns each (Chan, Golub and LeVeque, "Algorithms for computing the sample
// variance", 1983): mu = sum s_b / n, M2 = sum_b (M2_b + 32 (s_b / 32 - mu)^2), var = M2 / n, n = 32 ln_parts,
// sums in block order. Up to 32 partials (K <= 1024) of a 16-byte aligned array are loaded at once into registers,
// 16 bytes per load (only the P / 2 loads the row has: the partials are re-read by every column tile, so their volume
// is what this costs), and summed twice; more, or an array that is only 8-byte aligned, are read twice from memory
// 8 bytes at a time (the same sums in the same order). Every consumer (register epilogues, split-K reduction) forms
// the statistics with this one function.
__device__ __forceinline__ float2 ln_row(const GemmArgs &a, uint32_t gm) {
    if (a.ln_parts == 0) return ((const float2 *)a.ln_stats)[gm];
    const uint32_t P = a.ln_parts;
    const float2 *pp = (const float2 *)a.ln_stats + (uint64_t)gm * P;
    const float inv_n = 1.f / (32.f * (float)P);
    float s = 0.f, m2 = 0.f;
    if (P <= 32 && P % 2 == 0 && ((uintptr_t)a.ln_stats & 15u) == 0) {
        const uint32_t last = P / 2 - 1;             // wave-uniform: the branches below skip whole loads
        float4 q[16];
#pragma unroll
        for (int h = 0; h < 16; ++h)
            if ((uint32_t)h <= last) q[h] = ((const float4 *)pp)[h];
#pragma unroll
        for (int h = 0; h < 16; ++h)
            if ((uint32_t)h <= last) s += q[h].x + q[h].z;
        const float mu = s * inv_n;
#pragma unroll
        for (int h = 0; h < 16; ++h) {
            if ((uint32_t)h > last) continue;
            const float d0 = fmaf(q[h].x, 1.f / 32.f, -mu), d1 = fmaf(q[h].z, 1.f / 32.f, -mu);
            m2 += fmaf(32.f * d0, d0, q[h].y) + fmaf(32.f * d1, d1, q[h].w);
        }
        return make_float2(mu, sh_fast_rsq(fmaf(m2, inv_n, a.ln_eps)));
    }
    for (uint32_t b = 0; b < P; b += 2) s += pp[b].x + (b + 1 < P ? pp[b + 1].x : 0.f);
    const float mu = s * inv_n;
    for (uint32_t b = 0; b < P; b += 2) {
        const float2 q0 = pp[b], q1 = b + 1 < P ? pp[b + 1] : make_float2(32.f * mu, 0.f);
        const float d0 = fmaf(q0.x, 1.f / 32.f, -mu), d1 = fmaf(q1.x, 1.f / 32.f, -mu);
        m2 += fmaf(32.f * d0, d0, q0.y) + fmaf(32.f * d1, d1, q1.y);
    }
    return make_float2(mu, sh_fast_rsq(fmaf(m2, inv_n, a.ln_eps)));
}

// A wavefront's rows' fold factors (r and r mu of rows mrow + 32 i + r32), formed once at the start of a tile so
// the loads overlap its first DMAs and the epilogue waits on nothing: lane l forms rows mrow + l + 64 k, and each
// lane takes its rows' factors from those lanes.
template <int FM>
struct LnRows { float r[FM], rm[FM]; };
template <int FM>
__device__ __forceinline__ LnRows<FM> ln_rows(const GemmArgs &a, uint32_t mrow) {
    constexpr int RPL = (FM + 1) / 2;                // rows formed per lane
    LnRows<FM> l;
    const int lane = threadIdx.x & 63, r32 = lane & 31;
    if (!a.ln_stats) {
#pragma unroll
        for (int i = 0; i < FM; ++i) { l.r[i] = 0.f; l.rm[i] = 0.f; }
        return l;
    }
    float2 st[RPL];
#pragma unroll
    for (int k = 0; k < RPL; ++k) st[k] = ln_row(a, min(mrow + 64 * k + lane, a.M - 1));
#pragma unroll
    for (int i = 0; i < FM; ++i) {                   // row 32 i + r32 was formed by lane 32 (i % 2) + r32, k = i / 2
        const float mu = __shfl(st[i / 2].x, 32 * (i % 2) + r32, 64), r = __shfl(st[i / 2].y, 32 * (i % 2) + r32, 64);
        l.r[i] = r;
        l.rm[i] = mu * r;
    }
    return l;
}

// LayerNorm folded into the product (sh_gemm_epi.ln_stats): p -> r p - (r mu) c + d in fp32, before the fp16
// rounding; the bias (d) is part of this step, so the chain below skips it. st = ln_row(a, gm).
__device__ __forceinline__ float ln_apply(const GemmArgs &a, float2 st, float p, uint32_t gn) {
    return fmaf(st.y, p, fmaf(-(st.x * st.y), a.ln_c[gn], ((const float *)a.bias)[gn]));
}

// Logical tile of block b -> (split, tile row, tile column). Dispatch deals workgroups round-robin over the
// XCDs, so block b becomes logical index (b % X) (T / X) + b / X: each XCD walks a contiguous run of the tile
// order and the operand panels it shares stay in that XCD's L2. The order is row-major, or (group_m > 1) in bands
// of group_m tile rows taken column by column, so the tiles an XCD runs at once span group_m row panels of X and
// a few column panels of W instead of every column panel (a bijection: a band's last, short one included).
__device__ __forceinline__ void tile_of(const GemmArgs &a, uint32_t b, uint32_t nblk, uint32_t &tm, uint32_t &tn, uint32_t &split) {
    uint32_t L = b;
    if (a.xcd_groups > 1) L = (b % a.xcd_groups) * (nblk / a.xcd_groups) + b / a.xcd_groups;
    const uint32_t per = a.tiles_m * a.tiles_n;
    split = L / per;
    const uint32_t l = L - split * per;
    if (a.group_m > 1) {
        const uint32_t band = l / (a.group_m * a.tiles_n), first = band * a.group_m;
        const uint32_t rows = min(a.group_m, a.tiles_m - first), w = l - band * a.group_m * a.tiles_n;
        tm = first + w % rows;
        tn = w / rows;
    } else {
        tm = l / a.tiles_n;
        tn = l % a.tiles_n;
    }
}

// Zero-filled stand-in read by the epilogue for operands a call does not have (never written).
__device__ __align__(64) uint32_t g_epi_zero[16];

__device__ __forceinline__ uint32_t swz(uint32_t r) { return (r ^ (r >> 3)) & 7u; }

template <int BM, int BN>
struct Cfg {
    static constexpr int TM = BM / 2, TN = BN / 2;         // wavefront sub-tile
    static constexpr int FM = TM / 32, FN = TN / 32;       // MFMA tiles per wavefront
    static constexpr int A_PER_T = BM * 8 / 256;           // 16-byte X chunks per thread per slice
    static constexpr size_t STAGE_BYTES = (size_t)(BM + BN) * BK * 2;
    static constexpr size_t LDS = (2 * STAGE_BYTES > (size_t)BM * BN * 2) ? 2 * STAGE_BYTES : (size_t)BM * BN * 2;
    static_assert(BM % 64 == 0 && BN % 64 == 0 && BN <= 256 && BM * 8 % 256 == 0, "tile");
};

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

// 8 halves starting at element (r, c) of a row-major [rows, ld] matrix, zero outside [0, rmax) x [0, cmax).
template <bool VEC>
__device__ __forceinline__ uint4 load8(const uint16_t *p, uint64_t ld, uint32_t r, uint32_t c, uint32_t rmax, uint32_t cmax) {
    if (VEC) {
        if (r < rmax && c < cmax) return *(const uint4 *)(p + (uint64_t)r * ld + c);
        return zero4();
    } else {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (r < rmax && c + e < cmax) ? p[(uint64_t)r * ld + c + e] : 0u;
        return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    }
}

__device__ __forceinline__ uint32_t comp(const uint4 &q, int i) { return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w; }

// The epilogue chain applied to one fp16 product value, each step rounded to fp16 exactly as the unfused
// library sequence sh_gemm -> (accumulate) -> sh_add_bias -> sh_gelu -> sh_add would store it:
// z = r16(z_old + p) [accumulate]; z = r16(z + bias); z = r16(gelu(z)); z = r16(z + residual).
__device__ __forceinline__ uint16_t epi_chain(const GemmArgs &a, uint16_t p, uint32_t gm, uint32_t gn) {
    float v = sh_dev_h2f(p);
    if (a.accumulate) v = sh_dev_h2f(sh_dev_f2h_rr(v + sh_dev_h2f(a.z[(uint64_t)gm * a.ldz + gn])));
    if (a.bias && !a.ln_stats) {
        const float b = a.bias_fp32 ? ((const float *)a.bias)[gn] : sh_dev_h2f(((const uint16_t *)a.bias)[gn]);
        v = sh_dev_h2f(sh_dev_f2h_rr(v + b));
    }
    if (a.act == SH_ACT_GELU) { const uint16_t h = sh_dev_f2h(v); v = sh_dev_h2f((uint16_t)sh_gelu_u32(h | ((uint32_t)h << 16))); }
    if (a.res) v += sh_dev_h2f(a.res[(uint64_t)gm * a.ldr + gn]);
    return sh_dev_f2h(v);
}

// The same chain on 8 consecutive columns, with z_old / bias / residual already loaded (16-byte chunks; an
// fp32 bias is b0:b1). fp16 + fp16 steps use packed fp16 adds, which round exactly like the fp32 form above.
__device__ __forceinline__ uint4 epi_chain8(const GemmArgs &a, uint4 q, const uint4 &zo, const uint4 &b0, const uint4 &b1,
                                            const uint4 &rq) {
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
    if (a.accumulate) {
#pragma unroll
        for (int p = 0; p < 4; ++p) w[p] = sh_hadd2(comp(zo, p), w[p]);
    }
    if (a.bias && !a.ln_stats) {
        if (a.bias_fp32) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const sh_h2 h = __builtin_bit_cast(sh_h2, w[p]);
                const uint4 &bb = p < 2 ? b0 : b1;
                const float lo = (float)h.x + __uint_as_float(comp(bb, (2 * p) & 3));
                const float hi = (float)h.y + __uint_as_float(comp(bb, (2 * p + 1) & 3));
                w[p] = (uint32_t)sh_dev_f2h_rr(lo) | ((uint32_t)sh_dev_f2h_rr(hi) << 16);
            }
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) w[p] = sh_hadd2(w[p], comp(b0, p));
        }
    }
    if (a.act == SH_ACT_GELU) {
#pragma unroll
        for (int p = 0; p < 4; ++p) w[p] = sh_gelu_u32(w[p]);
    }
    if (a.res) {
#pragma unroll
        for (int p = 0; p < 4; ++p) w[p] = sh_hadd2(w[p], comp(rq, p));
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Accumulators -> Z. Element (i, j, r) of a wavefront is tile row wm*TM + 32 i + 8 (r/4) + 4 g + r%4 and
// column wn*TN + 32 j + r32 (v_mfma_f32_32x32x16 output layout). Split-K: fp32 partials straight to the
// workspace. Otherwise the products are rounded to fp16 into an LDS copy of the tile (16-byte chunk c of row
// r stored at c ^ (r & 7)), then written as 16-byte row chunks through the epilogue chain. `sC` must be free.
template <int BM, int BN, bool VEC, bool SPLIT, int FM, int FN>
__device__ __forceinline__ void epilogue(const GemmArgs &a, sh_f16v (&acc)[FM][FN], uint32_t m0, uint32_t n0, uint32_t split, uint16_t *sC) {
    constexpr int TM = BM / 2, TN = BN / 2;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, r32 = lane & 31;
    if (SPLIT) {
        float *P = a.part + (uint64_t)split * a.M * a.N;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const uint32_t gn = n0 + wn * TN + j * 32 + r32;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t gm = m0 + wm * TM + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (gm < a.M && gn < a.N) P[(uint64_t)gm * a.N + gn] = acc[i][j][r];
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const uint32_t col = wn * TN + j * 32 + r32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = wm * TM + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                sC[row * BN + (((col >> 3) ^ (row & 7)) << 3) + (col & 7)] = sh_dev_f2h(acc[i][j][r]);
            }
            __builtin_amdgcn_sched_barrier(0);     // one accumulator tile at a time (register pressure)
        }
    __syncthreads();
    const bool plain = !a.accumulate && !a.bias && a.act == SH_ACT_NONE && !a.res;
    constexpr int CPR = BN / 8;             // 16-byte chunks per tile row
    if (VEC && plain) {
        for (int c = t; c < BM * CPR; c += 256) {
            const int row = c / CPR, ch = c % CPR;
            const uint32_t gm = m0 + row, gn = n0 + 8 * ch;
            if (gm < a.M && gn < a.N) *(uint4 *)(a.z + (uint64_t)gm * a.ldz + gn) = ((const uint4 *)sC)[row * CPR + (ch ^ (row & 7))];
        }
    } else if (VEC) {
        // Chunk c = t + 256 i of the tile, in batches of NB chunks: (1) every global operand of the batch is
        // loaded, branch-free, before any is used; (2) the fp16 products are read from LDS; (3) the chain runs;
        // (4) the stores go out. A batch waits for one memory latency, and no load waits behind a store. An
        // operand that is off is read from a 64-byte zero block (one cached line) and ignored.
        constexpr int ITER = BM * CPR / 256, CAP = BM * BN >= 256 * 256 ? 4 : 6;       // CAP: registers in flight
        constexpr int NB = ITER % CAP == 0 ? CAP : ITER % 4 == 0 ? 4 : ITER % 2 == 0 ? 2 : 1;
        static_assert(ITER * 256 == BM * CPR && ITER % NB == 0, "epilogue chunk split");
        const uint16_t *zero = (const uint16_t *)g_epi_zero;
        const uint16_t *zs = a.accumulate ? a.z : zero, *rs = a.res ? a.res : zero;
        const uint64_t ldzs = a.accumulate ? a.ldz : 0, ldrs = a.res ? a.ldr : 0;
        const uint32_t zcs = a.accumulate ? 1 : 0, rcs = a.res ? 1 : 0;
        const char *bs = a.bias ? (const char *)a.bias : (const char *)zero;
        const uint32_t besz = a.bias ? (a.bias_fp32 ? 4 : 2) : 0, b1off = (a.bias && a.bias_fp32) ? 16 : 0;
#pragma unroll 1
        for (int i0 = 0; i0 < ITER; i0 += NB) {
            uint4 q[NB], zo[NB], b0[NB], b1[NB], rq[NB];
            uint32_t gms[NB], gns[NB];
            bool ok[NB];
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int c = t + 256 * (i0 + j), row = c / CPR, ch = c % CPR;
                ok[j] = m0 + row < a.M && n0 + 8 * ch < a.N;
                gms[j] = ok[j] ? m0 + row : m0;
                gns[j] = ok[j] ? n0 + 8 * ch : n0;
                zo[j] = *(const uint4 *)(zs + gms[j] * ldzs + gns[j] * zcs);
                b0[j] = *(const uint4 *)(bs + gns[j] * besz);
                b1[j] = *(const uint4 *)(bs + gns[j] * besz + b1off);
                rq[j] = *(const uint4 *)(rs + gms[j] * ldrs + gns[j] * rcs);
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int c = t + 256 * (i0 + j), row = c / CPR, ch = c % CPR;
                q[j] = ((const uint4 *)sC)[row * CPR + (ch ^ (row & 7))];
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) q[j] = epi_chain8(a, q[j], zo[j], b0[j], b1[j], rq[j]);
#pragma unroll
            for (int j = 0; j < NB; ++j)
                if (ok[j]) *(uint4 *)(a.z + (uint64_t)gms[j] * a.ldz + gns[j]) = q[j];
        }
    } else {
        for (int c = t; c < BM * CPR; c += 256) {
            const int row = c / CPR, ch = c % CPR;
            const uint32_t gm = m0 + row, gn = n0 + 8 * ch;
            if (gm >= a.M || gn >= a.N) continue;
            const uint4 q = ((const uint4 *)sC)[row * CPR + (ch ^ (row & 7))];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (gn + e >= a.N) break;
                const uint16_t h = (uint16_t)(comp(q, e >> 1) >> (16 * (e & 1)));
                a.z[(uint64_t)gm * a.ldz + gn + e] = plain ? h : epi_chain(a, h, gm, gn + e);
            }
        }
    }
}

template <int BM, int BN, bool VEC, bool SPLIT, bool WT = false>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
    using C = Cfg<BM, BN>;
    extern __shared__ uint4 smem[];
    uint4 *sA = smem;                       // [2][BM * 8]
    uint4 *sB = smem + 2 * BM * 8;          // [2][BN * 8]

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, r32 = lane & 31;

    // workgroup -> (split, tile_m, tile_n)
    const uint32_t nblk = a.tiles_m * a.tiles_n * a.splits;
    uint32_t tm, tn, split;
    tile_of(a, blockIdx.x, nblk, tm, tn, split);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t kbeg = split * a.kps;
    const uint32_t kend = min(a.K, kbeg + a.kps);
    const int KT = kend > kbeg ? (int)((kend - kbeg + BK - 1) / BK) : 0;

    sh_f16v acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) acc[i][j] = sh_f16v{};

    uint4 ra[C::A_PER_T];
    uint4 rb[8];
    const bool bload = t < BN;                    // W: one 8 x 8 block per thread, BN blocks per slice
    const int bkb = t & 7, bnc = t >> 3;
    constexpr int B_PER_T = BN * 8 / 256;         // WT: 16-byte chunks of W^T rows per thread per slice

    auto gload = [&](int kt) {
        const uint32_t k0 = kbeg + (uint32_t)kt * BK;
#pragma unroll
        for (int i = 0; i < C::A_PER_T; ++i) {
            const int c = t + 256 * i, row = c >> 3, kc = c & 7;
            ra[i] = load8<VEC>(a.x, a.ldx, m0 + row, k0 + 8 * kc, a.M, kend);
        }
        if constexpr (WT) {                       // W^T [N, K]: rows of k, loaded like X
#pragma unroll
            for (int i = 0; i < B_PER_T; ++i) {
                const int c = t + 256 * i, n = c >> 3, kc = c & 7;
                rb[i] = load8<VEC>(a.w, a.ldw, n0 + n, k0 + 8 * kc, a.N, kend);
            }
        } else if (bload) {
#pragma unroll
            for (int r = 0; r < 8; ++r) rb[r] = load8<VEC>(a.w, a.ldw, k0 + 8 * bkb + r, n0 + 8 * bnc, kend, a.N);
        }
    };
    auto sstore = [&](int st) {
        uint4 *pa = sA + st * BM * 8;
#pragma unroll
        for (int i = 0; i < C::A_PER_T; ++i) {
            const int c = t + 256 * i, row = c >> 3, kc = c & 7;
            pa[row * 8 + (kc ^ swz(row))] = ra[i];
        }
        if constexpr (WT) {
            uint4 *pb = sB + st * BN * 8;
#pragma unroll
            for (int i = 0; i < B_PER_T; ++i) {
                const int c = t + 256 * i, n = c >> 3, kc = c & 7;
                pb[n * 8 + (kc ^ swz(n))] = rb[i];
            }
        } else if (bload) {
            uint4 *pb = sB + st * BN * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j) {         // W^T row n = 8 bnc + j holds column j of the block
                uint32_t o[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const uint32_t lo = comp(rb[2 * p], j >> 1), hi = comp(rb[2 * p + 1], j >> 1);
                    o[p] = (j & 1) ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
                }
                const int n = 8 * bnc + j;
                pb[n * 8 + (bkb ^ swz(n))] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    };
    auto compute = [&](int st) {
        const uint4 *pa = sA + st * BM * 8, *pb = sB + st * BN * 8;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t ch = 4 * g + s;
            sh_h8 af[C::FM], bf[C::FN];
#pragma unroll
            for (int i = 0; i < C::FM; ++i) {
                const uint32_t row = wm * C::TM + i * 32 + r32;
                af[i] = __builtin_bit_cast(sh_h8, pa[row * 8 + (ch ^ swz(row))]);
            }
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                const uint32_t n = wn * C::TN + j * 32 + r32;
                bf[j] = __builtin_bit_cast(sh_h8, pb[n * 8 + (ch ^ swz(n))]);
            }
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
#pragma unroll
                for (int j = 0; j < C::FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    if (KT > 0) {
        gload(0);
        sstore(0);
        __syncthreads();
        for (int kt = 0; kt < KT; ++kt) {
            if (kt + 1 < KT) gload(kt + 1);
            compute(kt & 1);
            if (kt + 1 < KT) sstore((kt + 1) & 1);
            __syncthreads();
        }
    }

    epilogue<BM, BN, VEC, SPLIT, C::FM, C::FN>(a, acc, m0, n0, split, (uint16_t *)smem);
}

// ---- v2: direct global -> LDS loads, W read through the LDS transpose unit ----------------------------
// For 16-byte-aligned operands with K % 64 == 0. Each 64-k slice of X (BM rows, k contiguous) and of W (64 rows,
// n contiguous: the caller's [K, N] layout) is copied HBM -> LDS by global_load_lds_dwordx4 (no VGPR staging);
// a wave's instruction fills 1 KB of consecutive LDS, so the XOR swizzles are applied by choosing which
// global chunk each lane fetches. STAGES slices are in flight: the loads of slice kt + STAGES - 1 are issued
// right after the barrier that opens slice kt, and the wait for slice kt only drains the older loads
// (vmcnt, in-order completion). The MFMA B operand (8 consecutive k of one column n per lane) comes from two
// ds_read_b64_tr_b16: in a group of 16 lanes, lane i supplies the 8-byte row segment W[k0 + i/4][n0 + 4 (i%4)]
// and receives W[k0 + e][n0 + lane%16] for e = 0..3. Rows of W are swizzled at 16-byte granularity
// (chunk c of row k at c ^ fW(k)) so the 4-row x 64-byte footprint of such a read hits distinct banks.
// Rows of X beyond M and columns of W beyond N are fetched from clamped (valid) addresses; they only feed
// outputs that are never stored.
template <int BM, int BN, int STAGES>
struct Cfg2 {
    static constexpr int TM = BM / 2, TN = BN / 2, FM = TM / 32, FN = TN / 32;
    static constexpr int XCH = BM * 8;               // 16-byte chunks per X slice
    static constexpr int WCPR = BN / 8;              // chunks per W row
    static constexpr int WCH = BK * WCPR;            // chunks per W slice
    static constexpr int XR = XCH / 256, WR = WCH / 256;
    static constexpr int LOADS = XR + WR;            // DMA instructions per wave per slice
    static constexpr size_t STAGE = (size_t)(XCH + WCH) * 16;
    static constexpr size_t LDS = STAGES * STAGE > (size_t)BM * BN * 2 ? STAGES * STAGE : (size_t)BM * BN * 2;
    static_assert(BM % 64 == 0 && BN % 64 == 0 && XCH % 256 == 0 && WCH % 256 == 0, "tile");
    static_assert(LOADS < 64 && LDS <= 160 * 1024, "resources");
};

template <int BN>
__device__ __forceinline__ uint32_t fw(uint32_t k) {
    return ((BN / 8) % 16 == 0) ? 4u * (k & 3u) : 4u * ((k >> 1) & 1u);
}

template <int BM, int BN, int STAGES, bool SPLIT, bool KTAIL = false>
__global__ __launch_bounds__(256) void k_gemm2(GemmArgs a) {
    using C = Cfg2<BM, BN, STAGES>;
    extern __shared__ uint4 smem[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, r32 = lane & 31;

    const uint32_t nblk = a.tiles_m * a.tiles_n * a.splits;
    uint32_t tm, tn, split;
    tile_of(a, blockIdx.x, nblk, tm, tn, split);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t kbeg = split * a.kps;
    const uint32_t kend = min(a.K, kbeg + a.kps);
    const int KT = kend > kbeg ? (int)((kend - kbeg + (KTAIL ? BK - 1 : 0)) / BK) : 0;
    // KTAIL (K % 64 != 0): the last slice holds `rem` < 64 valid k (a multiple of 8); its X chunks and W rows
    // past kend are read from the zero block, so both operands are 0 there and add nothing
    const uint32_t rem = KT > 0 ? (kend - kbeg) - (uint32_t)(KT - 1) * BK : BK;
    const uint16_t *zero = (const uint16_t *)g_epi_zero;

    // per-lane source pointers of every DMA round (the k0 advance is added per slice), and whether the round's
    // chunk lies past kend in the last slice
    const uint16_t *xs[C::XR];
    const uint16_t *ws[C::WR];
    bool xpast[C::XR], wpast[C::WR];
#pragma unroll
    for (int r = 0; r < C::XR; ++r) {
        const uint32_t p = r * 256 + wave * 64 + lane, m = p >> 3, c = (p & 7) ^ swz(m);
        const uint32_t gm = min(m0 + m, a.M - 1);
        xs[r] = a.x + (uint64_t)gm * a.ldx + kbeg + 8 * c;
        xpast[r] = 8 * c >= rem;
    }
#pragma unroll
    for (int r = 0; r < C::WR; ++r) {
        const uint32_t p = r * 256 + wave * 64 + lane, k = p / C::WCPR, c = (p % C::WCPR) ^ fw<BN>(k);
        uint32_t gn = n0 + 8 * c;
        if (gn >= a.N) gn = a.N - 8;
        ws[r] = a.w + (uint64_t)(kbeg + k) * a.ldw + gn;
        wpast[r] = k >= rem;
    }
    const uint32_t lds0 = sh_lds_addr(smem);
    const uint32_t wave_off = (uint32_t)__builtin_amdgcn_readfirstlane(wave * 64 * 16);

    // DMA instruction d of the loads of k-slice `src` into LDS stage `stage`: X rounds first, then W rounds
    auto issue_one = [&](int d, int src, int stage) {
        const uint32_t st = lds0 + (uint32_t)stage * (uint32_t)C::STAGE;
        const bool last = KTAIL && src == KT - 1;
        if (d < C::XR) sh_lds_dma16(last && xpast[d] ? zero : xs[d] + (uint64_t)src * BK, st + d * 4096 + wave_off);
        else sh_lds_dma16(last && wpast[d - C::XR] ? zero : ws[d - C::XR] + (uint64_t)src * BK * a.ldw,
                       st + C::XCH * 16 + (d - C::XR) * 4096 + wave_off);
    };

    sh_f16v acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) acc[i][j] = sh_f16v{};

    // lane constants of the fragment reads
    const int q = lane >> 4, iq = lane & 15;
    uint32_t aoff[C::FM];
#pragma unroll
    for (int i = 0; i < C::FM; ++i) aoff[i] = (uint32_t)(wm * C::TM + i * 32 + r32);

    // Prologue: slices 0 .. STAGES-2. Every iteration then issues exactly LOADS DMAs (slices past the end are
    // clamped to the last slice and land in a stage nobody reads again), so the wait is a constant count.
    if (KT > 0) {
#pragma unroll
        for (int s = 0; s < STAGES - 1; ++s)
#pragma unroll
            for (int d = 0; d < C::LOADS; ++d) issue_one(d, min(s, KT - 1), s);
    }

    constexpr int NM = C::FM * C::FN;                 // MFMAs per k-substep
    constexpr int MT = 4 * NM;                        // per slice
    for (int kt = 0; kt < KT; ++kt) {
        sh_wait_vmcnt<(STAGES - 2) * C::LOADS>();        // this slice has landed (own wave) ...
        __syncthreads();                              // ... for every wave; the oldest stage is free again
        const int kn = min(kt + STAGES - 1, KT - 1);  // slice whose loads are spread over this slice's MFMAs ...
        const int kst = (kt + STAGES - 1) % STAGES;   // ... into the stage freed by the barrier above
        const uint32_t st = lds0 + (uint32_t)(kt % STAGES) * (uint32_t)C::STAGE;
        const uint4 *X = (const uint4 *)((const char *)smem + (uint32_t)(kt % STAGES) * (uint32_t)C::STAGE);
        const uint32_t wbase = st + C::XCH * 16;
        // fragments of k-substep s (16 k): A from X rows (one 16-byte read), B from two transpose reads
        auto load_frags = [&](int s, sh_h8 (&af)[C::FM], sh_h8 (&bf)[C::FN]) {
#pragma unroll
            for (int i = 0; i < C::FM; ++i) {
                const uint32_t m = aoff[i];
                af[i] = __builtin_bit_cast(sh_h8, X[m * 8 + ((2 * s + g) ^ swz(m))]);
            }
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                const uint32_t n = (uint32_t)(wn * C::TN + j * 32 + 16 * (q & 1) + 4 * (iq & 3));
                const uint32_t k0 = 16 * s + 8 * g + (iq >> 2), k1 = k0 + 4;
                const sh_s4 lo = sh_ds_read_tr(wbase + k0 * (BN * 2) + 16 * ((n >> 3) ^ fw<BN>(k0)) + 2 * (n & 7));
                const sh_s4 hi = sh_ds_read_tr(wbase + k1 * (BN * 2) + 16 * ((n >> 3) ^ fw<BN>(k1)) + 2 * (n & 7));
                bf[j] = __builtin_bit_cast(sh_h8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            }
        };
        sh_h8 af[2][C::FM], bf[2][C::FN];
        load_frags(0, af[0], bf[0]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // the reads of substep s + 1 are issued before the MFMAs of substep s (fenced so the scheduler
            // cannot sink them next to their consumers): their LDS latency hides under s's MFMAs
            if (s < 3) load_frags(s + 1, af[(s + 1) & 1], bf[(s + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
#pragma unroll
                for (int j = 0; j < C::FN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s & 1][i], bf[s & 1][j], acc[i][j], 0, 0, 0);
                    // DMA d goes out after MFMA number floor(d * MT / LOADS): loads trickle under the MFMAs
                    const int gi = s * NM + i * C::FN + j;
#pragma unroll
                    for (int d = 0; d < C::LOADS; ++d)
                        if (d * MT / C::LOADS == gi) { __builtin_amdgcn_sched_barrier(0); issue_one(d, kn, kst); __builtin_amdgcn_sched_barrier(0); }
                }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    sh_wait_vmcnt<0>();     // the clamped tail loads must land before the tile is staged in the same LDS
    __syncthreads();     // every wavefront is done with the slices before the tile is staged in the same LDS
    epilogue<BM, BN, true, SPLIT, C::FM, C::FN>(a, acc, m0, n0, split, (uint16_t *)smem);
}

// ---- epilogue from registers (Z^T accumulator layout) ------------------------------------------------------
// Kernels that pass the MFMA operands swapped (first = W fragment, second = X fragment) hold every 32 x 32
// accumulator as a block of Z^T: lane l has row l % 32 of Z and columns 8 q + 4 g + e in register 4 q + e
// (q, e = 0..3, g = l / 32). One permlane32 swap per register pair hands each lane 8 consecutive columns of its
// row, which pass through the epilogue chain and leave as one 16-byte store: no LDS staging and no barrier.
// The products are the same k-ordered sums as with the operands in X, W order (the tests check every
// configuration stores the same bits). The helpers take the wavefront's position (wm, wn) in the 2 x 2 grid of
// (BM/2) x (BN/2) sub-tiles.

// x's upper 32 lanes <-> y's lower 32 lanes (v_permlane32_swap_b32).
__device__ __forceinline__ void swap_halves(uint32_t &x, uint32_t &y) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
    x = r[0];
    y = r[1];
}

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {     // (fp32 values rounded to fp16 once more)
    asm volatile("" : "+v"(lo), "+v"(hi));           // (as sh_dev_f2h_rr: no conversion folded into the producer)
    return __builtin_bit_cast(uint32_t, sh_h2{(_Float16)lo, (_Float16)hi});
}

// The LayerNorm fold on a wavefront's Z^T accumulators (block (i, j) of lane l: the row of ln's entry i, columns
// ncol + 32 j + 8 q + 4 g + e in register 4 q + e), in place, before they are rounded.
template <int FM, int FN, bool OFF32 = false>
__device__ __forceinline__ void ln_fold_zt(const GemmArgs &a, sh_f16v (&acc)[FM][FN], const LnRows<FM> &ln, uint32_t ncol) {
    const int lane = threadIdx.x & 63, g = lane >> 5;
    const float *rr = ln.r, *rm = ln.rm;
    const float *d = (const float *)a.bias;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        float cj[16], dj[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t n = min(ncol + 32 * j + 8 * q + 4 * g, a.N - 4);
            // (OFF32: scalar base plus a 32-bit byte offset, N < 2^24)
            const float4 c4 = OFF32 ? *(const float4 *)((const char *)a.ln_c + n * 4u) : *(const float4 *)(a.ln_c + n);
            const float4 d4 = OFF32 ? *(const float4 *)((const char *)d + n * 4u) : *(const float4 *)(d + n);
            cj[4 * q] = c4.x; cj[4 * q + 1] = c4.y; cj[4 * q + 2] = c4.z; cj[4 * q + 3] = c4.w;
            dj[4 * q] = d4.x; dj[4 * q + 1] = d4.y; dj[4 * q + 2] = d4.z; dj[4 * q + 3] = d4.w;
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(rr[i], acc[i][j][r], fmaf(-rm[i], cj[r], dj[r]));
    }
}

// Row partials of a wavefront's finished chunks (Z^T layout: chunk (i, j, p) of a lane is row rbase + 32 i + r32,
// columns cbase + 32 j + 16 p + 8 g): for each row and each 32-column block, the sum s of its 32 stored fp16 values
// and M2 = sum (v - s / 32)^2 (two passes in fp32; lanes g = 0, 1 hold 16 values each), written as a float2 to
// stats_out[row][block] (the consumer combines a row's blocks with ln_row). Stores the same bits in every
// register-epilogue tile (the same 32 values, the same order).
template <int FM, int FN, bool OFF32 = false>
__device__ __forceinline__ void stats_zt(const GemmArgs &a, const uint4 (&q)[FM][FN][2], uint32_t rbase, uint32_t cbase) {
    const int lane = threadIdx.x & 63, g = lane >> 5, r32 = lane & 31;
    const uint32_t P = a.N / 32;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const uint32_t row = rbase + 32 * i + r32;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            float x[16], sum = 0.f;
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const sh_h2 h = __builtin_bit_cast(sh_h2, comp(q[i][j][p], w));
                    x[8 * p + 2 * w] = (float)h.x;
                    x[8 * p + 2 * w + 1] = (float)h.y;
                }
#pragma unroll
            for (int e = 0; e < 16; ++e) sum += x[e];
            sum += __shfl_xor(sum, 32, 64);
            const float mb = sum * (1.f / 32.f);
            float m2 = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) { const float d = x[e] - mb; m2 = fmaf(d, d, m2); }
            m2 += __shfl_xor(m2, 32, 64);
            const uint32_t col = cbase + 32 * j;
            if (g == 0 && row < a.M && col < a.N) {
                if constexpr (OFF32)           // (M N / 4 bytes of partials < 4 GiB: the launch checks it)
                    *(float2 *)((char *)a.stats_out + (__umul24(row, P) + col / 32) * 8u) = make_float2(sum, m2);
                else
                    ((float2 *)a.stats_out)[(uint64_t)row * P + col / 32] = make_float2(sum, m2);
            }
        }
    }
}

// 8 consecutive fp16 products of row block i, column block j, half p of one lane, in the Z^T layout above.
// Both 16-byte chunks (p = 0, 1) of the 32 x 32 block come out of the same four swaps.
template <int FM, int FN>
__device__ __forceinline__ void zt_chunks(const sh_f16v (&acc)[FM][FN], int i, int j, uint4 (&q)[2]) {
    uint32_t P[4][2];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        P[u][0] = pack_h2(acc[i][j][4 * u], acc[i][j][4 * u + 1]);
        P[u][1] = pack_h2(acc[i][j][4 * u + 2], acc[i][j][4 * u + 3]);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        swap_halves(P[2 * p][0], P[2 * p + 1][0]);
        swap_halves(P[2 * p][1], P[2 * p + 1][1]);
        q[p] = make_uint4(P[2 * p][0], P[2 * p][1], P[2 * p + 1][0], P[2 * p + 1][1]);
    }
}

// The epilogue chain on a tile's chunks in place (q from zt_chunks of every block; chunk (i, j, p) of a lane is
// row m0 + wm TM + 32 i + r32, columns n0 + wn TN + 32 j + 16 p + 8 g). Converting every accumulator first
// halves the registers the epilogue holds. For the common chains (fp16 or no bias, optional residual) every
// operand load of the tile is issued in one batch, so the epilogue waits for one memory latency.
template <int BM, int BN, int FM, int FN>
__device__ __forceinline__ void chain_chunks(const GemmArgs &a, uint4 (&q)[FM][FN][2], uint32_t m0, uint32_t n0, int wm, int wn) {
    constexpr int TM = BM / 2, TN = BN / 2;
    const int lane = threadIdx.x & 63, g = lane >> 5, r32 = lane & 31;
    if (!a.accumulate && (!a.bias || a.ln_stats) && !a.res && a.act == SH_ACT_NONE) return;
    if (!a.accumulate && (!(a.bias && a.bias_fp32) || a.ln_stats)) {
        uint4 bq[FN][2];
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint32_t gn = n0 + wn * TN + 32 * j + 16 * p + 8 * g, gc = min(gn, a.N - 8);
                bq[j][p] = (a.bias && !a.ln_stats) ? *(const uint4 *)((const uint16_t *)a.bias + gc) : zero4();
            }
        uint4 rq[FM][FN][2];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const uint32_t gm = m0 + wm * TM + 32 * i + r32;
            const uint64_t rowr = (uint64_t)min(gm, a.M - 1) * a.ldr;
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const uint32_t gn = n0 + wn * TN + 32 * j + 16 * p + 8 * g, gc = min(gn, a.N - 8);
                    rq[i][j][p] = a.res ? *(const uint4 *)(a.res + rowr + gc) : zero4();
                }
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int p = 0; p < 2; ++p) q[i][j][p] = epi_chain8(a, q[i][j][p], zero4(), bq[j][p], zero4(), rq[i][j][p]);
        return;
    }
    // z_old (accumulate) or a 32-byte fp32 bias per chunk: one (row block, column block) at a time
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const uint32_t gm = m0 + wm * TM + 32 * i + r32;
        const uint32_t gmc = min(gm, a.M - 1);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            uint4 zo[2], b0[2], b1[2], rq[2];
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint32_t gn = n0 + wn * TN + 32 * j + 16 * p + 8 * g, gc = min(gn, a.N - 8);
                zo[p] = a.accumulate ? *(const uint4 *)(a.z + (uint64_t)gmc * a.ldz + gc) : zero4();
                if (a.bias && a.bias_fp32) {
                    b0[p] = *(const uint4 *)((const float *)a.bias + gc);
                    b1[p] = *(const uint4 *)((const float *)a.bias + gc + 4);
                } else {
                    b0[p] = a.bias ? *(const uint4 *)((const uint16_t *)a.bias + gc) : zero4();
                    b1[p] = zero4();
                }
                rq[p] = a.res ? *(const uint4 *)(a.res + (uint64_t)gmc * a.ldr + gc) : zero4();
            }
#pragma unroll
            for (int p = 0; p < 2; ++p) q[i][j][p] = epi_chain8(a, q[i][j][p], zo[p], b0[p], b1[p], rq[p]);
        }
    }
}

// Store a finished tile's chunks (origin m0, n0).
template <int BM, int BN, int FM, int FN>
__device__ __forceinline__ void store_all(const GemmArgs &a, const uint4 (&q)[FM][FN][2], uint32_t m0, uint32_t n0, int wm, int wn) {
    constexpr int TM = BM / 2, TN = BN / 2;
    const int lane = threadIdx.x & 63, g = lane >> 5, r32 = lane & 31;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint32_t gm = m0 + wm * TM + 32 * i + r32, gn = n0 + wn * TN + 32 * j + 16 * p + 8 * g;
                if (gm < a.M && gn < a.N) *(uint4 *)(a.z + (uint64_t)gm * a.ldz + gn) = q[i][j][p];
            }
}

// Store a wavefront's finished block (TM x TN at rbase, cbase) through LDS: 32 rows at a time, its Z^T chunks (chunk
// (i, j, p) of a lane: row 32 i + r32, columns 32 j + 16 p + 8 g) go to a row-major copy in LDS that only this
// wavefront writes (`slots`: its NSLOT 1 KB DMA slots, slot s at slots + SSTRIDE s, in a stage no wavefront
// reads any more), then each store instruction writes 64 consecutive 16-byte chunks of those rows (whole row segments
// of the block) instead of 32 rows x 32 bytes. The residual of the epilogue chain is added to the row chunks here
// (the chain up to it was applied to q without it; the same fp16 adds, so the same bits). LDS instructions of
// one wavefront execute in order, so no barrier is involved. Chunk lin of the row-major copy sits at lin ^ (row &
// 15) within its 16-chunk line: the staging writes (lanes 0-31 at rows 0-31, CPRW chunks apart) then hit 16
// distinct 16-byte bank groups per 16 lanes instead of 16 / gcd(CPRW, 16) of them (4- to 16-way conflicts), and
// the reads of 16 consecutive chunks stay a permutation of one line.
// The slots may span NSTG free stages of the ring: slot s is slot s % NSLOT of stage (first + s / NSLOT) mod nst,
// stages stage_bytes apart from `ring` (the ring base plus the wavefront's offset in a slot).
// OFF32: Z and the residual span less than 4 GiB from their bases, and rows and leading dimensions are below 2^24
// (the launch checks both): each lane's store and load addresses are the tensor's base (scalar registers) plus a
// 32-bit byte offset from a 24-bit multiply-add, instead of 64-bit address arithmetic.
template <int TM, int TN, int FM, int FN, int NSLOT, int SSTRIDE, int NSTG = 1, bool OFF32 = false>
__device__ __forceinline__ void store_wave_staged(const GemmArgs &a, const uint4 (&q)[FM][FN][2], uint32_t rbase, uint32_t cbase,
                                                  char *ring, uint32_t first, uint32_t nst, uint32_t stage_bytes) {
    constexpr int CPRW = TN / 8, HALF = 32 * CPRW, STEPS = HALF / 64;
    static_assert(HALF % 64 == 0 && STEPS <= NSLOT * NSTG, "32 rows of the block fit in the wavefront's slots");
    const int lane = threadIdx.x & 63, g = lane >> 5, r32 = lane & 31;
    auto phys = [](int lin) { return lin ^ ((lin / CPRW) & 15); };      // stays inside lin's 16-chunk line
    auto slot = [&](int sl) -> char * {
        uint32_t st = first + (uint32_t)(sl / NSLOT);
        if (st >= nst) st -= nst;
        return ring + (size_t)st * stage_bytes + (size_t)(sl % NSLOT) * SSTRIDE;
    };
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        uint4 rq[STEPS];
#pragma unroll
        for (int u = 0; u < STEPS; ++u) {                // residual row chunks first: their latency overlaps the staging
            const int lin = u * 64 + lane, row = lin / CPRW, c = lin % CPRW;
            const uint32_t gm = min(rbase + 32 * i + row, a.M - 1), gn = min(cbase + 8 * c, a.N - 8);
            if constexpr (OFF32)
                rq[u] = a.res ? *(const uint4 *)((const char *)a.res + (__umul24(gm, (uint32_t)a.ldr) + gn) * 2u) : zero4();
            else
                rq[u] = a.res ? *(const uint4 *)(a.res + (uint64_t)gm * a.ldr + gn) : zero4();
        }
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int pl = phys(r32 * CPRW + 4 * j + 2 * p + g);
                *(uint4 *)(slot(pl / 64) + (pl % 64) * 16) = q[i][j][p];
            }
#pragma unroll
        for (int u = 0; u < STEPS; ++u) {
            const int lin = u * 64 + lane, row = lin / CPRW, c = lin % CPRW;
            uint4 v = *(const uint4 *)(slot(u) + (phys(lin) % 64) * 16);
            if (a.res) v = make_uint4(sh_hadd2(v.x, rq[u].x), sh_hadd2(v.y, rq[u].y), sh_hadd2(v.z, rq[u].z), sh_hadd2(v.w, rq[u].w));
            const uint32_t gm = rbase + 32 * i + row, gn = cbase + 8 * c;
            if constexpr (OFF32) {
                if (gm < a.M && gn < a.N) *(uint4 *)((char *)a.z + (__umul24(gm, (uint32_t)a.ldz) + gn) * 2u) = v;
            } else {
                if (gm < a.M && gn < a.N) *(uint4 *)(a.z + (uint64_t)gm * a.ldz + gn) = v;
            }
        }
    }
}

// Split-K: the fp32 partial tile straight from the Z^T layout, 4 consecutive columns (16 bytes) per store.
template <int BM, int BN, int FM, int FN>
__device__ __forceinline__ void store_partials_zt(const GemmArgs &a, const sh_f16v (&acc)[FM][FN], uint32_t m0, uint32_t n0,
                                                  uint32_t split, int wm, int wn) {
    constexpr int TM = BM / 2, TN = BN / 2;
    const int lane = threadIdx.x & 63, g = lane >> 5, r32 = lane & 31;
    float *P = a.part + (uint64_t)split * a.M * a.N;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t gm = m0 + wm * TM + 32 * i + r32, gn = n0 + wn * TN + 32 * j + 8 * u + 4 * g;
                if (gm < a.M && gn < a.N)
                    *(float4 *)(P + (uint64_t)gm * a.N + gn) =
                        make_float4(acc[i][j][4 * u], acc[i][j][4 * u + 1], acc[i][j][4 * u + 2], acc[i][j][4 * u + 3]);
            }
}

// X row swizzle of a slice. 32-k slices have 64-byte LDS rows (4 chunks of 16 B): chunk c of row m is stored at
// c ^ ((m >> 2) & 3), so the 16 rows read by 16 lanes of one ds_read_b128 cover 16 distinct 16-byte bank groups.
// 64-k slices have 128-byte rows, swizzled as in k_gemm2.
__device__ __forceinline__ uint32_t sx4(uint32_t m) { return (m >> 2) & 3u; }
template <int SK>
__device__ __forceinline__ uint32_t xswz(uint32_t m) { return SK == 32 ? sx4(m) : swz(m); }

// ---- v5: LDS-lean tiles, MFMAs interleaved one by one with the LDS reads and DMAs ---------------------------
// Four wavefronts (2 x 2, one per SIMD), each owning a (BM/2) x (BN/2) block of Z^T accumulators (MFMA operands
// swapped, epilogue straight from registers: see above). SK-wide k-slices (32 or 64) flow through an
// NST-stage LDS ring filled by global_load_lds_dwordx4; one barrier per slice. Within a slice the work is cut
// into one segment per 16-k substep: segment s issues the fragment reads of substep s and its share of the
// DMAs of slice kt + NST - 1, each placed between two MFMAs of substep s - 1 (the MFMAs of a slice's last
// substep run in the next slice's first segment, after its barrier). The order is fixed in source with
// sched_barrier fences: every 32-cycle MFMA has at most a few other instructions between it and the next, so
// the MFMA pipe never waits on a burst of reads, and each read is issued several MFMAs before its first use.
// W is read either in the caller's [K, N] layout (LDS transpose reads, as k_gemm2) or, with WT, as W^T [N, K]
// (rows of k like X: plain 16-byte LDS reads, half the LDS read cost). The k order per lane is k_gemm2's
// (substep s, lane group g -> 8-k chunk 2 s + g), so every configuration stores the same bits.
// PRE: the epilogue's bias row and residual are loaded into registers at the start of the last slice, so the
// epilogue does not wait a memory latency after the last MFMA (register budget permitting).
// f(std::integral_constant<int, I>{}) for I = 0 .. N - 1, unrolled at compile time
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &f, std::integer_sequence<int, I...>) { (f(std::integral_constant<int, I>{}), ...); }
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) { static_for_impl(f, std::make_integer_sequence<int, N>{}); }

template <int BM, int BN, int SK, int NST, bool WT>
struct Cfg5 {
    static constexpr int TM = BM / 2, TN = BN / 2, FM = TM / 32, FN = TN / 32, NS = SK / 16;
    static constexpr int XCPR = SK / 8;                  // 16-byte chunks per k-row (X rows; W^T rows)
    static constexpr int WCPR = BN / 8;                  // chunks per n-row of W ([K, N] layout)
    static constexpr int XCH = BM * XCPR, WCH = BN * XCPR;
    static constexpr int XR = XCH / 256, WR = WCH / 256, LOADS = XR + WR;
    static constexpr int RD = FM + FN * (WT ? 1 : 2);    // LDS read instructions per substep
    static constexpr int NM = FM * FN;                   // MFMAs per substep
    static constexpr size_t STAGE = (size_t)(XCH + WCH) * 16;
    static constexpr size_t LDS = NST * STAGE;
    static_assert(BM % 64 == 0 && BN % 64 == 0 && (SK == 32 || SK == 64) && XCH % 256 == 0 && WCH % 256 == 0, "tile");
    static_assert(NST >= 2 && LOADS * (NST - 2) < 64 && LDS <= 160 * 1024, "resources");
};

// KG = 2: in-workgroup split-K. Two groups of four wavefronts (512 threads, two rings) compute one tile; group g
// runs the slices of K range g (a.kps each, both ranges the same length, so both groups pass the same barriers)
// through its own ring, then group 1 hands its fp32 accumulators to group 0 through its ring and group 0 adds them
// (first range + second, as the reduction adds two partials) and runs the unsplit epilogue: the bits of the
// two-partial path without the partials' HBM traffic or the reduction launch. One workgroup holds a CU, with two
// wavefronts per SIMD where a tile grid of one workgroup per CU would leave one.
// EPI (unsplit builds of the encoder's tiles): the epilogue a call has, fixed at compile time so its flag tests
// and the code behind them drop out (the same arithmetic and bits as EPI = 0, which reads every flag from the
// arguments): 1 = LayerNorm fold with the fp32 row d, then GELU; 2 = LayerNorm fold with d; 3 = fp16 bias, residual
// and row partials; 4 = fp16 bias; 5 = fp16 bias, then GELU; 6 = fp16 bias and residual; 7 = none (the product
// alone). gemm_epi_kind picks it for a call; the arguments' own fields still hold the pointers.
enum { EPI_ANY = 0, EPI_FOLD_GELU = 1, EPI_FOLD = 2, EPI_BIAS_RES_STATS = 3, EPI_BIAS = 4, EPI_BIAS_GELU = 5,
       EPI_BIAS_RES = 6, EPI_PLAIN = 7, EPI_KINDS = 8 };
template <int EPI>
__device__ __forceinline__ GemmArgs gemm_epi_spec(const GemmArgs &in) {
    GemmArgs a = in;
    if constexpr (EPI == EPI_FOLD_GELU || EPI == EPI_FOLD) {
        a.accumulate = 0; a.res = nullptr; a.bias_fp32 = 1; a.stats_out = nullptr;
        a.act = EPI == EPI_FOLD_GELU ? SH_ACT_GELU : SH_ACT_NONE;
        __builtin_assume(a.bias != nullptr);      // (the launch picks these builds only for calls that have them)
        __builtin_assume(a.ln_stats != nullptr);
    } else if constexpr (EPI == EPI_BIAS_RES_STATS) {
        a.accumulate = 0; a.ln_stats = nullptr; a.ln_parts = 0; a.bias_fp32 = 0; a.act = SH_ACT_NONE;
        __builtin_assume(a.bias != nullptr);
        __builtin_assume(a.res != nullptr);
        __builtin_assume(a.stats_out != nullptr);
    } else if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_GELU || EPI == EPI_BIAS_RES) {
        a.accumulate = 0; a.ln_stats = nullptr; a.ln_parts = 0; a.bias_fp32 = 0; a.stats_out = nullptr;
        a.act = EPI == EPI_BIAS_GELU ? SH_ACT_GELU : SH_ACT_NONE;
        __builtin_assume(a.bias != nullptr);
        if constexpr (EPI == EPI_BIAS_RES) __builtin_assume(a.res != nullptr);
        else a.res = nullptr;
    } else if constexpr (EPI == EPI_PLAIN) {
        a.accumulate = 0; a.ln_stats = nullptr; a.ln_parts = 0; a.bias = nullptr; a.bias_fp32 = 0; a.stats_out = nullptr;
        a.act = SH_ACT_NONE; a.res = nullptr;
    }
    return a;
}

template <int BM, int BN, int SK, int NST, bool WT, int MINW, bool SPLIT, bool PRE, int KG = 1, int EPI = EPI_ANY>
__global__ __launch_bounds__(256 * KG, MINW) void k_gemm5(GemmArgs a_in) {
    static_assert(EPI == EPI_ANY || (!SPLIT && KG == 1 && !WT), "epilogue builds are unsplit");
    const GemmArgs a = gemm_epi_spec<EPI>(a_in);
    using C = Cfg5<BM, BN, SK, NST, WT>;
    constexpr int TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN, NS = C::NS, XCPR = C::XCPR;
    static_assert(KG == 1 || (KG == 2 && !SPLIT && 2 * C::LDS <= 160 * 1024 && 16 * FN * 1024 <= (int)C::LDS), "k groups");
    extern __shared__ uint4 smem[];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane((t >> 6) & 3);
    const int grp = KG > 1 ? __builtin_amdgcn_readfirstlane(t >> 8) : 0;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, r32 = lane & 31;
    uint4 *const ring = smem + (size_t)grp * (C::LDS / 16);     // this group's stages

    const uint32_t nblk = a.tiles_m * a.tiles_n * (KG > 1 ? 1u : a.splits);
    uint32_t tm, tn, split;
    tile_of(a, blockIdx.x, nblk, tm, tn, split);
    if constexpr (KG > 1) split = (uint32_t)grp;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t kbeg = split * a.kps;
    const uint32_t kend = min(a.K, kbeg + a.kps);
    const int KT = kend > kbeg ? (int)((kend - kbeg) / SK) : 0;

    // per-lane DMA sources of every round; rows past M (W^T rows past N, W columns past N) read clamped valid
    // addresses and only feed outputs that are never stored
    const uint16_t *xs[C::XR];
    const uint16_t *ws[C::WR];
#pragma unroll
    for (int r = 0; r < C::XR; ++r) {
        const uint32_t p = r * 256 + wave * 64 + lane, m = p / XCPR, c = (p % XCPR) ^ xswz<SK>(m);
        xs[r] = a.x + (uint64_t)min(m0 + m, a.M - 1) * a.ldx + kbeg + 8 * c;
    }
#pragma unroll
    for (int r = 0; r < C::WR; ++r) {
        const uint32_t p = r * 256 + wave * 64 + lane;
        if constexpr (WT) {
            const uint32_t n = p / XCPR, c = (p % XCPR) ^ xswz<SK>(n);
            ws[r] = a.w + (uint64_t)min(n0 + n, a.N - 1) * a.ldw + kbeg + 8 * c;
        } else {
            const uint32_t k = p / C::WCPR, c = (p % C::WCPR) ^ fw<BN>(k);
            uint32_t gn = n0 + 8 * c;
            if (gn >= a.N) gn = a.N - 8;
            ws[r] = a.w + (uint64_t)(kbeg + k) * a.ldw + gn;
        }
    }
    const uint64_t wadv = WT ? (uint64_t)SK : (uint64_t)SK * a.ldw;
    const uint32_t lds0 = sh_lds_addr(ring);
    const uint32_t wave_off = (uint32_t)wave * 1024u;
    // epilogue builds (the launch checks the leading dimensions): the same addresses as a wave-uniform base per operand
    // (scalar registers, advanced by the slice) plus each lane's 32-bit byte offset from it, which is >= 0 since the
    // clamped rows and columns never fall below the tile's first (no 64-bit vector add per DMA)
    constexpr bool OFF32 = EPI != EPI_ANY;
    const char *const xb = (const char *)(a.x + (uint64_t)m0 * a.ldx + kbeg);
    const char *const wb = WT ? (const char *)(a.w + (uint64_t)n0 * a.ldw + kbeg) : (const char *)(a.w + (uint64_t)kbeg * a.ldw + n0);
    uint32_t xo[C::XR], wo[C::WR];
#pragma unroll
    for (int r = 0; r < C::XR; ++r) xo[r] = (uint32_t)((const char *)xs[r] - xb);
#pragma unroll
    for (int r = 0; r < C::WR; ++r) wo[r] = (uint32_t)((const char *)ws[r] - wb);
    auto dma = [&](int d, int src, int stage) {          // DMA instruction d of slice `src` into `stage`
        const uint32_t st = lds0 + (uint32_t)stage * (uint32_t)C::STAGE;
        if constexpr (OFF32) {
            if (d < C::XR) sh_lds_dma16_s(xb + (uint64_t)src * SK * 2, xo[d], st + d * 4096 + wave_off);
            else sh_lds_dma16_s(wb + (uint64_t)src * wadv * 2, wo[d - C::XR], st + C::XCH * 16 + (d - C::XR) * 4096 + wave_off);
        } else {
            if (d < C::XR) sh_lds_dma16(xs[d] + (uint64_t)src * SK, st + d * 4096 + wave_off);
            else sh_lds_dma16(ws[d - C::XR] + (uint64_t)src * wadv, st + C::XCH * 16 + (d - C::XR) * 4096 + wave_off);
        }
    };

    // fragment reads: instruction r of substep s (X fragments first, then W fragments, one or two each)
    const int q = lane >> 4, iq = lane & 15;
    // W fragments: WT -> wf (one 16-byte read); [K, N] layout -> two transpose reads into wl / wh, joined at use
    sh_h8 xf[2][FM], wf[2][WT ? FN : 1];
    sh_s4 wl[2][WT ? 1 : FN], wh[2][WT ? 1 : FN];
    auto wfrag = [&](int buf, int j) -> sh_h8 {
        if constexpr (WT) return wf[buf][j];
        else return __builtin_bit_cast(sh_h8, __builtin_shufflevector(wl[buf][j], wh[buf][j], 0, 1, 2, 3, 4, 5, 6, 7));
    };
    // [K, N] layout: each transpose read's LDS address in stage 0, per (substep, column block, half), formed once;
    // a read adds its stage as an immediate offset
    uint32_t wra[WT ? 1 : NS][WT ? 1 : FN][2];
    if constexpr (!WT) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const uint32_t n = (uint32_t)(wn * TN + j * 32 + 16 * (q & 1) + 4 * (iq & 3));
                    const uint32_t k = 16 * s + 8 * g + (iq >> 2) + 4 * half;
                    wra[s][j][half] = lds0 + C::XCH * 16 + k * (BN * 2) + 16 * ((n >> 3) ^ fw<BN>(k)) + 2 * (n & 7);
                }
    }
    auto read = [&](int stage, int s, int r, int buf) {
        const uint32_t sb = (uint32_t)stage * (uint32_t)C::STAGE;
        const uint32_t c = (uint32_t)(2 * s + g);
        if (r < FM) {
            const uint4 *X = (const uint4 *)((const char *)ring + sb);
            const uint32_t m = (uint32_t)(wm * TM + r * 32 + r32);
            xf[buf][r] = __builtin_bit_cast(sh_h8, X[m * XCPR + (c ^ xswz<SK>(m))]);
        } else if constexpr (WT) {
            const int j = r - FM;
            const uint4 *W = (const uint4 *)((const char *)ring + sb + C::XCH * 16);
            const uint32_t n = (uint32_t)(wn * TN + j * 32 + r32);
            wf[buf][j] = __builtin_bit_cast(sh_h8, W[n * XCPR + (c ^ xswz<SK>(n))]);
        } else {
            const int j = (r - FM) >> 1, half = (r - FM) & 1;
            const sh_s4 v = sh_ds_read_tr(wra[WT ? 0 : s][WT ? 0 : j][half] + sb);
            if (!half) wl[buf][j] = v;
            else wh[buf][j] = v;
        }
    };

    sh_f16v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = sh_f16v{};
#pragma unroll
    for (int b = 0; b < 2; ++b) {              // the "previous substep" of slice 0 multiplies zeros: acc stays +0
#pragma unroll
        for (int i = 0; i < FM; ++i) xf[b][i] = sh_h8{};
        if constexpr (WT) {
#pragma unroll
            for (int j = 0; j < FN; ++j) wf[b][j] = sh_h8{};
        } else {
#pragma unroll
            for (int j = 0; j < FN; ++j) { wl[b][j] = sh_s4{}; wh[b][j] = sh_s4{}; }
        }
    }

    // epilogue operands loaded early (PRE): fp16 bias chunks and residual chunks of this lane's outputs
    // (the largest tiles keep their registers for the accumulators: no early loads there)
    // (unsplit tiles are stored through each wavefront's DMA slots, and the residual is added there: no early load)
    // (the staging may use every stage but the last slice's: NST - 1 stages of LOADS 1 KB slots per wavefront)
    // (a tile that holds a CU alone, MINW = 1, has the registers to load the residual early even when staged)
    constexpr bool STAGED = !SPLIT && 4 * TN <= 64 * C::LOADS * (NST - 1);
    constexpr bool PRE_B = PRE && FM * FN <= 12, PRE_RES = PRE && FM * FN <= 6 && (!STAGED || (MINW == 1 && KG == 1));
    uint4 bq[PRE_B ? FN : 1][2], rq[PRE_RES ? FM : 1][PRE_RES ? FN : 1][2];
    // (a GEMM that also writes row partials adds the residual in the chain, before them)
    const bool has_stats = EPI == EPI_BIAS_RES_STATS ? true : EPI != EPI_ANY ? false : a.stats_out != nullptr;
    const bool has_res = (EPI == EPI_BIAS_RES_STATS || EPI == EPI_BIAS_RES) ? true : EPI != EPI_ANY ? false : a.res != nullptr;
    const bool stage_res = STAGED && !PRE_RES && !has_stats;
    const bool pre_ok = PRE_B && grp == 0 && !a.accumulate && !(a.bias && a.bias_fp32) && (PRE_RES || stage_res || !has_res);
    auto prefetch = [&]() {
#pragma unroll
        for (int j = 0; j < (PRE_B ? FN : 0); ++j)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint32_t gc = min(n0 + wn * TN + 32 * j + 16 * p + 8 * g, a.N - 8);
                if constexpr (OFF32) bq[j][p] = a.bias ? *(const uint4 *)((const char *)a.bias + gc * 2u) : zero4();
                else bq[j][p] = a.bias ? *(const uint4 *)((const uint16_t *)a.bias + gc) : zero4();
            }
        if constexpr (PRE_RES) {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const uint64_t rowr = (uint64_t)min(m0 + wm * TM + 32 * i + r32, a.M - 1) * a.ldr;
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const uint32_t gc = min(n0 + wn * TN + 32 * j + 16 * p + 8 * g, a.N - 8);
                        rq[i][j][p] = a.res ? *(const uint4 *)(a.res + rowr + gc) : zero4();
                    }
            }
        }
    };

    if (KT > 0) {
#pragma unroll
        for (int s = 0; s < NST - 1; ++s)
#pragma unroll
            for (int d = 0; d < C::LOADS; ++d) dma(d, min(s, KT - 1), s);
    }
    // the rows' fold factors: their partials are loaded after the first DMAs, so the two latencies overlap (loads
    // complete in issue order, so the wait for the partials also sees those DMAs land)
    __builtin_amdgcn_sched_barrier(0);
    const LnRows<FM> lnw = ln_rows<FM>(a, m0 + wm * TM);
    // slice kt, held in ring stage st = kt % NST, fixed at compile time: the loop below is unrolled by the ring's
    // stages, so every fragment read is a per-lane register plus an immediate offset (no vector add per read)
    auto slice = [&](int kt, auto stc) __attribute__((always_inline)) {
        constexpr int st = decltype(stc)::value, nst = (st + NST - 1) % NST;
        sh_wait_vmcnt<(NST - 2) * C::LOADS>();           // slice kt landed (this wave's share) ...
        sh_wait_lgkm0();                                 // ... and this wave's reads of slice kt - 1 are done
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();                    // every share landed; the stage of slice kt - 1 is free
        __builtin_amdgcn_sched_barrier(0);
        if (PRE_B && kt == KT - 1 && pre_ok) prefetch();
        const int nsrc = min(kt + NST - 1, KT - 1);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int cur = s & 1, prv = cur ^ 1;
            // segment s: MFMA q of the previous substep, then read q (if any), then DMA q (if any)
#pragma unroll
            for (int qm = 0; qm < C::NM || qm < C::RD; ++qm) {
                if (qm < C::NM) {            // column-block major: the first MFMAs need the first reads
                    const int j = qm / FM, i = qm % FM;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wfrag(prv, j), xf[prv][i], acc[i][j], 0, 0, 0);
                }
                if (qm < C::RD) read(st, s, qm, cur);
                // this segment's DMAs (s * LOADS / NS .. (s + 1) * LOADS / NS) after the first reads
#pragma unroll
                for (int d = s * C::LOADS / NS; d < (s + 1) * C::LOADS / NS; ++d)
                    if (d - s * C::LOADS / NS == qm) dma(d, nsrc, nst);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    int kt0 = 0;
    for (; kt0 + NST <= KT; kt0 += NST)
        static_for<NST>([&](auto stc) __attribute__((always_inline)) { slice(kt0 + decltype(stc)::value, stc); });
    static_for<NST - 1>([&](auto stc) __attribute__((always_inline)) {
        if (kt0 + decltype(stc)::value < KT) slice(kt0 + decltype(stc)::value, stc);
    });
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wfrag((NS - 1) & 1, j), xf[(NS - 1) & 1][i], acc[i][j], 0, 0, 0);
    if constexpr (KG > 1) {
        sh_wait_vmcnt<0>();          // the clamped tail DMAs into the rings have landed ...
        __syncthreads();             // ... for every wavefront, and every read of group 1's ring is done
        // per row block i of fragments: 16 FN KB of group 1's ring, lane-contiguous 16-byte slots
        float4 *park = (float4 *)((char *)smem + C::LDS) + wave * (FN * 4 * 64) + lane;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            if (grp == 1) {
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        park[(j * 4 + e) * 64] = make_float4(acc[i][j][4 * e], acc[i][j][4 * e + 1], acc[i][j][4 * e + 2], acc[i][j][4 * e + 3]);
            }
            __syncthreads();
            if (grp == 0) {
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float4 v = park[(j * 4 + e) * 64];
                        acc[i][j][4 * e] += v.x; acc[i][j][4 * e + 1] += v.y;
                        acc[i][j][4 * e + 2] += v.z; acc[i][j][4 * e + 3] += v.w;
                    }
            }
            if (i + 1 < FM) __syncthreads();          // group 0 has read the block before group 1 overwrites it
        }
        if (grp == 1) return;        // no barrier follows: group 0 stores through its own ring
    }
    if constexpr (SPLIT) {
        store_partials_zt<BM, BN, FM, FN>(a, acc, m0, n0, split, wm, wn);
    } else {
        if (a.ln_stats) ln_fold_zt<FM, FN, OFF32>(a, acc, lnw, n0 + wn * TN);
        uint4 qc[FM][FN][2];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) zt_chunks<FM, FN>(acc, i, j, qc[i][j]);
        GemmArgs an = a;
        if (stage_res) an.res = nullptr;             // the residual is added to the staged row chunks
        if (PRE_B && pre_ok && KT > 0) {
            if (an.bias || an.res || an.act != SH_ACT_NONE) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int p = 0; p < 2; ++p)
                            qc[i][j][p] = epi_chain8(an, qc[i][j][p], zero4(), bq[PRE_B ? j : 0][p], zero4(),
                                                     PRE_RES ? rq[PRE_RES ? i : 0][PRE_RES ? j : 0][p] : zero4());
            }
        } else {
            chain_chunks<BM, BN, FM, FN>(an, qc, m0, n0, wm, wn);
        }
        if (has_stats) stats_zt<FM, FN, OFF32>(a, qc, m0 + wm * TM, n0 + wn * TN);
        if constexpr (STAGED) {
            // every stage but slice KT - 1's holds no slice any more (only the clamped tail DMAs, each wavefront's
            // into its own slots): their last reads were slices <= KT - 2, finished before slice KT - 1's barrier
            sh_wait_vmcnt<0>();                      // this wavefront's tail DMAs have landed
            constexpr int NSTG = (4 * TN + 64 * C::LOADS - 1) / (64 * C::LOADS);      // stages the block needs
            GemmArgs as = a;
            if (!stage_res) as.res = nullptr;        // already added in the chain
            store_wave_staged<TM, TN, FM, FN, C::LOADS, 4096, NSTG, EPI != EPI_ANY>(as, qc, m0 + wm * TM, n0 + wn * TN,
                                                                     (char *)smem + (size_t)wave * 1024, (uint32_t)(KT % NST),
                                                                     (uint32_t)NST, (uint32_t)C::STAGE);
        } else {
            store_all<BM, BN, FM, FN>(a, qc, m0, n0, wm, wn);
        }
    }
    sh_wait_vmcnt<0>();      // no DMA may still target this workgroup's LDS when it exits
}

// ---- v6: W given transposed ([N, K], k contiguous), large tiles, any 2-D wavefront grid -------------------
// For callers that hold W^T (weights transposed once, as the encoder does): both operands are rows of k, so both
// MFMA fragments come from plain 16-byte LDS reads (no transpose reads) and both DMA streams fetch whole k-row
// segments with one swizzle. The tile is BM x BN over a WGM x WGN grid of wavefronts (4, 8 or 12 of them), so a
// CU can hold a 256 x 384 tile whose operand feed, (BM + BN) x 2 bytes per k, stays within what one CU's
// vector-memory path delivers at the MFMA rate (a 128 x 192 tile needs 1.7x more per FLOP). Slices of SK k
// flow through an NST-stage DMA ring with one barrier per slice; as in k_gemm5 each 16-k substep's fragment
// reads and DMAs sit one by one between the MFMAs of the previous substep. Same k order per lane as every
// other direct-to-LDS kernel (chunk 2 s + g), so the same bits. Epilogue straight from the Z^T accumulators.
template <int BM, int BN, int WGM, int WGN, int SK, int NST>
struct Cfg6 {
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int TM = BM / WGM, TN = BN / WGN, FM = TM / 32, FN = TN / 32, NS = SK / 16;
    static constexpr int XCPR = SK / 8;                  // 16-byte chunks per k-row segment of a slice
    static constexpr int XCH = BM * XCPR, WCH = BN * XCPR;
    static constexpr int XR = XCH / NT, WR = WCH / NT, LOADS = XR + WR;
    static constexpr int RPR = NT / XCPR;                // rows one DMA round covers
    static constexpr int RD = FM + FN, NM = FM * FN;
    static constexpr size_t STAGE = (size_t)(XCH + WCH) * 16;
    static constexpr size_t LDS = NST * STAGE;
    static_assert(TM % 32 == 0 && TN % 32 == 0 && (SK == 32 || SK == 64) && XCH % NT == 0 && WCH % NT == 0, "tile");
    // the row swizzle of a k-row segment is the same in every DMA round (rows advance by a multiple of its period)
    static_assert(RPR % (SK == 64 ? 64 : 16) == 0, "DMA rounds must keep the row swizzle");
    static_assert(NST >= 2 && LOADS * (NST - 2) < 64 && LDS <= 160 * 1024 && NT <= 1024, "resources");
};

// DB: fragments double-buffered and interleaved with the previous substep's MFMAs (one wavefront per SIMD);
// without DB each substep reads its fragments, then runs its MFMAs, and the second wavefront of the SIMD covers
// the read latency (eight-wavefront tiles, whose accumulators leave no room for a second fragment set).
template <int BM, int BN, int WGM, int WGN, int SK, int NST, int MINW, bool SPLIT, bool PRE, bool DB = true>
__global__ __launch_bounds__(64 * WGM * WGN, MINW) void k_gemm6(GemmArgs a) {
    using C = Cfg6<BM, BN, WGM, WGN, SK, NST>;
    constexpr int TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN, NS = C::NS, XCPR = C::XCPR, NT = C::NT;
    extern __shared__ uint4 smem[];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WGN, wn = wave % WGN, g = lane >> 5, r32 = lane & 31;

    const uint32_t nblk = a.tiles_m * a.tiles_n * a.splits;
    uint32_t tm, tn, split;
    tile_of(a, blockIdx.x, nblk, tm, tn, split);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t kbeg = split * a.kps;
    const uint32_t kend = min(a.K, kbeg + a.kps);
    const int KT = kend > kbeg ? (int)((kend - kbeg) / SK) : 0;

    // DMA: round r, lane chunk p = r NT + 64 wave + lane is row r RPR + p0 / XCPR, 16-byte chunk (p0 % XCPR) ^ swizzle
    // (the same in every round); rows past M (N) read row M - 1 (N - 1): valid memory feeding unstored outputs
    const uint32_t p0 = (uint32_t)(wave * 64 + lane), row0 = p0 / XCPR, cg = (p0 % XCPR) ^ xswz<SK>(row0);
    const uint16_t *xbase = a.x + kbeg + 8 * cg, *wbase = a.w + kbeg + 8 * cg;   // a.w holds W^T [N, K]
    const uint32_t lds0 = sh_lds_addr(smem);
    const uint32_t wave_off = (uint32_t)wave * 1024u;
    auto dma = [&](int d, int src, int stage) {          // DMA instruction d of slice `src` into `stage`
        const uint32_t st = lds0 + (uint32_t)stage * (uint32_t)C::STAGE;
        if (d < C::XR) {
            const uint32_t m = min(m0 + (uint32_t)(d * C::RPR) + row0, a.M - 1);
            sh_lds_dma16(xbase + (uint64_t)m * a.ldx + (uint32_t)src * SK, st + d * NT * 16 + wave_off);
        } else {
            const uint32_t n = min(n0 + (uint32_t)((d - C::XR) * C::RPR) + row0, a.N - 1);
            sh_lds_dma16(wbase + (uint64_t)n * a.ldw + (uint32_t)src * SK, st + C::XCH * 16 + (d - C::XR) * NT * 16 + wave_off);
        }
    };
    constexpr int NB = DB ? 2 : 1;
    sh_h8 xf[NB][FM], wf[NB][FN];
    auto read = [&](int stage, int s, int r, int buf) {  // fragment read r of substep s: X fragments, then W^T
        const char *sb = (const char *)smem + (uint32_t)stage * (uint32_t)C::STAGE;
        const uint32_t c = (uint32_t)(2 * s + g);
        if (r < FM) {
            const uint32_t m = (uint32_t)(wm * TM + r * 32 + r32);
            xf[buf][r] = __builtin_bit_cast(sh_h8, ((const uint4 *)sb)[m * XCPR + (c ^ xswz<SK>(m))]);
        } else {
            const uint32_t n = (uint32_t)(wn * TN + (r - FM) * 32 + r32);
            wf[buf][r - FM] = __builtin_bit_cast(sh_h8, ((const uint4 *)(sb + C::XCH * 16))[n * XCPR + (c ^ xswz<SK>(n))]);
        }
    };

    sh_f16v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = sh_f16v{};
#pragma unroll
    for (int b = 0; b < NB; ++b) {             // the "previous substep" of slice 0 multiplies zeros: acc stays +0
#pragma unroll
        for (int i = 0; i < FM; ++i) xf[b][i] = sh_h8{};
#pragma unroll
        for (int j = 0; j < FN; ++j) wf[b][j] = sh_h8{};
    }

    // PRE: the bias row (and, for small per-wave blocks, the residual) loaded at the start of the last slice
    // (unsplit tiles of up to 6 blocks per wavefront are stored through each wavefront's DMA slots, and the residual
    // is added there: no early load; larger blocks leave no registers for the staging)
    constexpr bool STAGED = !SPLIT && 4 * TN <= 64 * C::LOADS && FM * FN <= 6;
    constexpr bool PRE_B = PRE, PRE_RES = PRE && FM * FN <= 6 && !STAGED;
    uint4 bq[PRE_B ? FN : 1][2], rq[PRE_RES ? FM : 1][PRE_RES ? FN : 1][2];
    const bool stage_res = STAGED && !a.stats_out;       // (row partials need the residual in the chain)
    const bool pre_ok = !SPLIT && PRE_B && !a.accumulate && !(a.bias && a.bias_fp32) && (PRE_RES || stage_res || !a.res);
    auto prefetch = [&]() {
#pragma unroll
        for (int j = 0; j < (PRE_B ? FN : 0); ++j)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint32_t gc = min(n0 + wn * TN + 32 * j + 16 * p + 8 * g, a.N - 8);
                bq[j][p] = a.bias ? *(const uint4 *)((const uint16_t *)a.bias + gc) : zero4();
            }
        if constexpr (PRE_RES) {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const uint64_t rowr = (uint64_t)min(m0 + wm * TM + 32 * i + r32, a.M - 1) * a.ldr;
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const uint32_t gc = min(n0 + wn * TN + 32 * j + 16 * p + 8 * g, a.N - 8);
                        rq[i][j][p] = a.res ? *(const uint4 *)(a.res + rowr + gc) : zero4();
                    }
            }
        }
    };

    if (KT > 0) {
#pragma unroll
        for (int s = 0; s < NST - 1; ++s)
#pragma unroll
            for (int d = 0; d < C::LOADS; ++d) dma(d, min(s, KT - 1), s);
    }
    // the rows' fold factors: their partials are loaded after the first DMAs, so the two latencies overlap (loads
    // complete in issue order, so the wait for the partials also sees those DMAs land)
    __builtin_amdgcn_sched_barrier(0);
    const LnRows<FM> lnw = ln_rows<FM>(a, m0 + wm * TM);
    for (int kt = 0; kt < KT; ++kt) {
        sh_wait_vmcnt<(NST - 2) * C::LOADS>();           // slice kt landed (this wave's share) ...
        sh_wait_lgkm0();                                 // ... and this wave's reads of slice kt - 1 are done
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();                    // every share landed; the stage of slice kt - 1 is free
        __builtin_amdgcn_sched_barrier(0);
        if (kt == KT - 1 && pre_ok) prefetch();
        const int st = kt % NST, nsrc = min(kt + NST - 1, KT - 1), nst = (kt + NST - 1) % NST;
        if constexpr (DB) {
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const int cur = s & 1, prv = cur ^ 1;
#pragma unroll
                for (int qm = 0; qm < C::NM || qm < C::RD; ++qm) {
                    if (qm < C::NM) {            // column-block major: the first MFMAs need the first reads
                        const int j = qm / FM, i = qm % FM;
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[prv][j], xf[prv][i], acc[i][j], 0, 0, 0);
                    }
                    if (qm < C::RD) read(st, s, qm, cur);
#pragma unroll
                    for (int d = s * C::LOADS / NS; d < (s + 1) * C::LOADS / NS; ++d)
                        if (d - s * C::LOADS / NS == qm) dma(d, nsrc, nst);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        } else {
#pragma unroll
            for (int d = 0; d < C::LOADS; ++d) dma(d, nsrc, nst);
#pragma unroll
            for (int s = 0; s < NS; ++s) {
#pragma unroll
                for (int r = 0; r < C::RD; ++r) read(st, s, r, 0);
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[0][j], xf[0][i], acc[i][j], 0, 0, 0);
            }
        }
    }
    if constexpr (DB) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < FM; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[(NS - 1) & 1][j], xf[(NS - 1) & 1][i], acc[i][j], 0, 0, 0);
    }

    // lane chunk (i, j, p): row m0 + wm TM + 32 i + r32, columns n0 + wn TN + 32 j + 16 p + 8 g
    if constexpr (SPLIT) {
        float *P = a.part + (uint64_t)split * a.M * a.N;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t gm = m0 + wm * TM + 32 * i + r32, gn = n0 + wn * TN + 32 * j + 8 * u + 4 * g;
                    if (gm < a.M && gn < a.N)
                        *(float4 *)(P + (uint64_t)gm * a.N + gn) =
                            make_float4(acc[i][j][4 * u], acc[i][j][4 * u + 1], acc[i][j][4 * u + 2], acc[i][j][4 * u + 3]);
                }
    } else {
        if constexpr (FM * FN <= 6) {                    // (the configurations that apply the fold unsplit)
            if (a.ln_stats) ln_fold_zt<FM, FN>(a, acc, lnw, n0 + wn * TN);
        }
        uint4 qc[FM][FN][2];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) zt_chunks<FM, FN>(acc, i, j, qc[i][j]);
        const bool has_res = a.res && !stage_res;        // staged tiles add the residual to their row chunks
        const bool any = a.accumulate || (a.bias && !a.ln_stats) || has_res || a.act != SH_ACT_NONE;
        GemmArgs an = a;
        if (stage_res) an.res = nullptr;
        if (any) {
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const uint32_t gmc = min(m0 + wm * TM + 32 * i + r32, a.M - 1);
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const uint32_t gc = min(n0 + wn * TN + 32 * j + 16 * p + 8 * g, a.N - 8);
                        uint4 zo = zero4(), b0 = zero4(), b1 = zero4(), rr = zero4();
                        if (pre_ok && KT > 0) {
                            b0 = bq[PRE_B ? j : 0][p];
                            if constexpr (PRE_RES) rr = rq[i][j][p];
                            else if (has_res) rr = *(const uint4 *)(a.res + (uint64_t)gmc * a.ldr + gc);
                        } else {
                            if (a.accumulate) zo = *(const uint4 *)(a.z + (uint64_t)gmc * a.ldz + gc);
                            if (a.bias && a.bias_fp32) {
                                b0 = *(const uint4 *)((const float *)a.bias + gc);
                                b1 = *(const uint4 *)((const float *)a.bias + gc + 4);
                            } else if (a.bias) {
                                b0 = *(const uint4 *)((const uint16_t *)a.bias + gc);
                            }
                            if (has_res) rr = *(const uint4 *)(a.res + (uint64_t)gmc * a.ldr + gc);
                        }
                        qc[i][j][p] = epi_chain8(an, qc[i][j][p], zo, b0, b1, rr);
                    }
            }
        }
        if constexpr (FM * FN <= 6) {                    // (larger blocks: no registers left; never chosen for them)
            if (a.stats_out) stats_zt<FM, FN>(a, qc, m0 + wm * TM, n0 + wn * TN);
        }
        if constexpr (STAGED) {
            // stage KT % NST holds no slice (only the clamped tail DMAs, each wavefront's into its own slots)
            sh_wait_vmcnt<0>();                          // this wavefront's tail DMAs have landed
            GemmArgs as = a;
            if (!stage_res) as.res = nullptr;            // already added in the chain
            store_wave_staged<TM, TN, FM, FN, C::LOADS, NT * 16>(as, qc, m0 + wm * TM, n0 + wn * TN,
                                                                  (char *)smem + (size_t)wave * 1024, (uint32_t)(KT % NST),
                                                                  (uint32_t)NST, (uint32_t)C::STAGE);
        } else {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const uint32_t gm = m0 + wm * TM + 32 * i + r32, gn = n0 + wn * TN + 32 * j + 16 * p + 8 * g;
                        if (gm < a.M && gn < a.N) *(uint4 *)(a.z + (uint64_t)gm * a.ldz + gn) = qc[i][j][p];
                    }
        }
    }
    sh_wait_vmcnt<0>();      // no DMA may still target this workgroup's LDS when it exits
}

// Sum of the split partials in split order, then the epilogue chain. Item = 8 columns (VEC) or 1.
template <bool VEC>
// One item per thread in 64-thread workgroups: a split-K output is usually small (M of a few hundred), and
// single-wave workgroups spread its items over every CU.
__global__ __launch_bounds__(64) void k_splitk_reduce(GemmArgs a, ShDiv div, uint32_t per_row, uint32_t items) {
    const uint32_t it = blockIdx.x * 64u + threadIdx.x;
    if (it >= items) return;
    const uint32_t gm = sh_div(it, div), cc = it - gm * per_row;
    const uint64_t plane = (uint64_t)a.M * a.N;
    constexpr int W = VEC ? 8 : 1;
    const uint32_t gn = VEC ? 8 * cc : cc;
    // v = 0, then v += partial_0, partial_1, ... in split order. The loads of SB splits are issued before the
    // adds that use them (one memory latency per SB splits, not per split); a split past a.splits reads
    // element 0 and adds +0, which leaves every sum as it was (after its first add v is never -0).
    constexpr int SB = 4;
    float v[W];
#pragma unroll
    for (int e = 0; e < W; ++e) v[e] = 0.f;
    const float *base = a.part + (uint64_t)gm * a.N + gn;
    for (uint32_t s = 0; s < a.splits; s += SB) {
        float u[SB][W];
#pragma unroll
        for (int q = 0; q < SB; ++q) {
            const bool in = s + q < a.splits;
            const float *p = in ? base + (uint64_t)(s + q) * plane : a.part;
            if (VEC) {
                const float4 u0 = *(const float4 *)p, u1 = *(const float4 *)(p + 4);
                u[q][0] = u0.x; u[q][1 % W] = u0.y; u[q][2 % W] = u0.z; u[q][3 % W] = u0.w;
                u[q][4 % W] = u1.x; u[q][5 % W] = u1.y; u[q][6 % W] = u1.z; u[q][7 % W] = u1.w;
            } else {
                u[q][0] = p[0];
            }
            const uint32_t mk = in ? 0xFFFFFFFFu : 0u;
#pragma unroll
            for (int e = 0; e < W; ++e) u[q][e] = __uint_as_float(__float_as_uint(u[q][e]) & mk);
        }
#pragma unroll
        for (int q = 0; q < SB; ++q)
#pragma unroll
            for (int e = 0; e < W; ++e) v[e] += u[q][e];
    }
    uint16_t out[W];
    if (a.ln_stats) {
        const float2 st = ln_row(a, gm);
#pragma unroll
        for (int e = 0; e < W; ++e) v[e] = ln_apply(a, st, v[e], gn + e);
    }
#pragma unroll
    for (int e = 0; e < W; ++e) out[e] = epi_chain(a, sh_dev_f2h_rr(v[e]), gm, gn + e);
    if (VEC && a.stats_out) {                        // 4 consecutive threads hold the 32 columns of one partial
        float x[W], sum = 0.f;
#pragma unroll
        for (int e = 0; e < W; ++e) { x[e] = sh_dev_h2f(out[e]); sum += x[e]; }
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        const float mb = sum * (1.f / 32.f);
        float m2 = 0.f;
#pragma unroll
        for (int e = 0; e < W; ++e) { const float d = x[e] - mb; m2 = fmaf(d, d, m2); }
        m2 += __shfl_xor(m2, 1, 64);
        m2 += __shfl_xor(m2, 2, 64);
        if ((cc & 3) == 0) ((float2 *)a.stats_out)[(uint64_t)gm * (a.N / 32) + cc / 4] = make_float2(sum, m2);
    }
    if (VEC) {
        uint32_t w4[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) w4[p] = (uint32_t)out[(2 * p) % W] | ((uint32_t)out[(2 * p + 1) % W] << 16);
        *(uint4 *)(a.z + (uint64_t)gm * a.ldz + gn) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    } else {
        a.z[(uint64_t)gm * a.ldz + gn] = out[0];
    }
}

// ---- host side ------------------------------------------------------------------------------------------
typedef void (*KernelFn)(GemmArgs);
// v2 entries need vec operands and K % 64 == 0; v1 entries take anything (scalar variants for small tiles).
// ktail: the kernel also takes K % 64 != 0 (vector operands; the last, partial k-slice reads zeros past K).
// wt: the configuration computes X . W from W^T ([N, K], sh_gemm_ex_wt) and only serves such calls; the
// register-staged configurations serve both layouts (wt_vec / wt_scalar: their W^T variants).
struct KCfg {
    int bm, bn, stages; bool v2; KernelFn vec[2], scalar[2]; size_t lds; float eff; bool attr_set; int threads = 256;
    bool ktail = false; KernelFn tail[2] = {nullptr, nullptr};     // the K % 64 != 0 variants (unsplit, split)
    bool wt = false; KernelFn wt_vec[2] = {nullptr, nullptr}, wt_scalar[2] = {nullptr, nullptr};
    bool reg = false;            // the unsplit epilogue applies a LayerNorm fold and writes row partials from registers
    KernelFn kg2 = nullptr;      // in-workgroup split-K over two equal K ranges (512 threads, two rings: 2 x lds bytes)
    KernelFn epi[EPI_KINDS] = {};     // unsplit builds with the epilogue fixed (k_gemm5 EPI)
};

#define SH_KCFG(BM, BN, EFF) { BM, BN, 2, false, { k_gemm<BM, BN, true, false>, k_gemm<BM, BN, true, true> }, \
                               { k_gemm<BM, BN, false, false>, k_gemm<BM, BN, false, true> }, Cfg<BM, BN>::LDS, EFF, false, 256, \
                               false, { nullptr, nullptr }, false, \
                               { k_gemm<BM, BN, true, false, true>, k_gemm<BM, BN, true, true, true> }, \
                               { k_gemm<BM, BN, false, false, true>, k_gemm<BM, BN, false, true, true> } }
#define SH_KCFG6(BM, BN, WGM, WGN, SK, NST, W, PRE, DB, EFF) \
    { BM, BN, NST, true, { k_gemm6<BM, BN, WGM, WGN, SK, NST, W, false, PRE, DB>, k_gemm6<BM, BN, WGM, WGN, SK, NST, W, true, PRE, DB> }, \
      { nullptr, nullptr }, Cfg6<BM, BN, WGM, WGN, SK, NST>::LDS, EFF, false, 64 * WGM * WGN, false, { nullptr, nullptr }, true, \
      { nullptr, nullptr }, { nullptr, nullptr }, Cfg6<BM, BN, WGM, WGN, SK, NST>::FM * Cfg6<BM, BN, WGM, WGN, SK, NST>::FN <= 6 }
#define SH_KCFG2(BM, BN, ST, EFF) { BM, BN, ST, true, { k_gemm2<BM, BN, ST, false>, k_gemm2<BM, BN, ST, true> }, \
                                    { nullptr, nullptr }, Cfg2<BM, BN, ST>::LDS, EFF, false, 256, true, \
                                    { k_gemm2<BM, BN, ST, false, true>, k_gemm2<BM, BN, ST, true, true> } }
#define SH_KCFG5(BM, BN, SK, NST, W, EFF) { BM, BN, NST, true, { k_gemm5<BM, BN, SK, NST, false, W, false, true>, \
                                              k_gemm5<BM, BN, SK, NST, false, W, true, true> }, \
                                            { nullptr, nullptr }, Cfg5<BM, BN, SK, NST, false>::LDS, EFF, false, 256, \
                                            false, { nullptr, nullptr }, false, { nullptr, nullptr }, { nullptr, nullptr }, true }
#define SH_KCFG5K(BM, BN, SK, NST, W, EFF) { BM, BN, NST, true, { k_gemm5<BM, BN, SK, NST, false, W, false, true>, \
                                               k_gemm5<BM, BN, SK, NST, false, W, true, true> }, \
                                             { nullptr, nullptr }, Cfg5<BM, BN, SK, NST, false>::LDS, EFF, false, 256, \
                                             false, { nullptr, nullptr }, false, { nullptr, nullptr }, { nullptr, nullptr }, true, \
                                             k_gemm5<BM, BN, SK, NST, false, 1, false, true, 2> }
// the same with the epilogue builds (the encoder's tiles)
#define SH_KCFG5_EPI(BM, BN, SK, NST, W) { nullptr, k_gemm5<BM, BN, SK, NST, false, W, false, true, 1, EPI_FOLD_GELU>, \
                                           k_gemm5<BM, BN, SK, NST, false, W, false, true, 1, EPI_FOLD>, \
                                           k_gemm5<BM, BN, SK, NST, false, W, false, true, 1, EPI_BIAS_RES_STATS>, \
                                           k_gemm5<BM, BN, SK, NST, false, W, false, true, 1, EPI_BIAS>, \
                                           k_gemm5<BM, BN, SK, NST, false, W, false, true, 1, EPI_BIAS_GELU>, \
                                           k_gemm5<BM, BN, SK, NST, false, W, false, true, 1, EPI_BIAS_RES>, \
                                           k_gemm5<BM, BN, SK, NST, false, W, false, true, 1, EPI_PLAIN> }
#define SH_KCFG5E(BM, BN, SK, NST, W, EFF) { BM, BN, NST, true, { k_gemm5<BM, BN, SK, NST, false, W, false, true>, \
                                               k_gemm5<BM, BN, SK, NST, false, W, true, true> }, \
                                             { nullptr, nullptr }, Cfg5<BM, BN, SK, NST, false>::LDS, EFF, false, 256, \
                                             false, { nullptr, nullptr }, false, { nullptr, nullptr }, { nullptr, nullptr }, true, \
                                             nullptr, SH_KCFG5_EPI(BM, BN, SK, NST, W) }
#define SH_KCFG5KE(BM, BN, SK, NST, W, EFF) { BM, BN, NST, true, { k_gemm5<BM, BN, SK, NST, false, W, false, true>, \
                                                k_gemm5<BM, BN, SK, NST, false, W, true, true> }, \
                                              { nullptr, nullptr }, Cfg5<BM, BN, SK, NST, false>::LDS, EFF, false, 256, \
                                              false, { nullptr, nullptr }, false, { nullptr, nullptr }, { nullptr, nullptr }, true, \
                                              k_gemm5<BM, BN, SK, NST, false, 1, false, true, 2>, SH_KCFG5_EPI(BM, BN, SK, NST, W) }
// eff = sustained fraction of the MFMA peak per CU measured for each tile on MI355X (tile-time model of
// est_time below); it only ranks the configurations.
KCfg g_cfgs[] = {
    SH_KCFG(256, 256, 0.22f),
    SH_KCFG(256, 128, 0.20f),
    SH_KCFG(128, 256, 0.20f),
    SH_KCFG(128, 192, 0.23f),
    SH_KCFG(128, 128, 0.22f),
    SH_KCFG(64, 64, 0.10f),
    SH_KCFG2(256, 256, 2, 0.35f),
    SH_KCFG2(256, 128, 3, 0.33f),
    SH_KCFG2(128, 192, 2, 0.30f),
    SH_KCFG2(128, 128, 2, 0.27f),
    SH_KCFG2(64, 64, 2, 0.12f),             // small tiles: many workgroups for small problems (latency-bound)
    SH_KCFG2(64, 64, 3, 0.13f),
    SH_KCFG2(64, 128, 2, 0.16f),
    SH_KCFG2(128, 64, 2, 0.16f),
    // LDS-lean tiles with MFMA / read / DMA interleaving (k_gemm5)
    SH_KCFG5(256, 192, 64, 2, 1, 0.38f),
    SH_KCFG5(128, 192, 64, 3, 1, 0.36f),
    SH_KCFG5KE(128, 192, 64, 2, 2, 0.36f),
    SH_KCFG5(128, 256, 64, 2, 1, 0.36f),
    // W^T operand (sh_gemm_ex_wt): 4 / 8 wavefronts, up to 256 x 384 tiles (k_gemm6)
    SH_KCFG6(256, 384, 2, 4, 64, 2, 2, false, false, 0.50f),
    SH_KCFG6(256, 384, 2, 4, 32, 4, 2, false, false, 0.50f),
    SH_KCFG6(256, 256, 2, 4, 64, 2, 2, false, true, 0.48f),
    SH_KCFG6(256, 256, 2, 4, 64, 2, 2, false, false, 0.48f),
    SH_KCFG6(256, 256, 2, 2, 32, 4, 1, true, true, 0.46f),
    SH_KCFG6(256, 192, 2, 2, 32, 4, 1, true, true, 0.44f),
    SH_KCFG6(128, 576, 2, 2, 32, 3, 1, false, true, 0.44f),
    SH_KCFG6(128, 192, 2, 2, 32, 6, 1, true, true, 0.40f),
    SH_KCFG6(128, 192, 2, 2, 32, 4, 2, true, true, 0.40f),
    SH_KCFG6(128, 192, 4, 2, 64, 3, 2, true, false, 0.40f),
    SH_KCFG6(64, 64, 2, 2, 32, 4, 2, false, true, 0.12f),        // small W^T tiles (small problems)
    SH_KCFG6(128, 64, 2, 2, 32, 4, 2, false, true, 0.16f),
    SH_KCFG6(64, 128, 2, 2, 32, 4, 2, false, true, 0.16f),
    SH_KCFG6(128, 128, 2, 2, 32, 4, 2, true, true, 0.25f),
    SH_KCFG5KE(128, 192, 32, 4, 2, 0.36f),      // two workgroups per CU with a deeper ring of 32-k slices
    SH_KCFG5(128, 128, 32, 4, 2, 0.30f),
    SH_KCFG5E(128, 192, 32, 4, 1, 0.36f),       // one workgroup per CU: residual and bias loaded during the last slice
};
#undef SH_KCFG
#undef SH_KCFG2
#undef SH_KCFG5
#undef SH_KCFG5E
#undef SH_KCFG5KE
#undef SH_KCFG5_EPI
#undef SH_KCFG5K
#undef SH_KCFG6
constexpr int kNumCfg = sizeof(g_cfgs) / sizeof(g_cfgs[0]);

int env_int(const char *name, int dflt) {
    const char *e = getenv(name);
    return (e && *e) ? atoi(e) : dflt;
}

// The K ranges a request for `want` splits launches: each range is a whole number of 64-k slices (kps), at
// most one range per slice, and no trailing range is empty. Every consumer of a split count (the cost model,
// sh_gemm_plan, the launch) goes through this, so what is priced and reported is what runs.
struct SplitK { uint32_t splits, kps; };
SplitK split_k(uint32_t K, uint32_t want) {
    const uint32_t k = std::max<uint32_t>(K, 1);
    const uint32_t s = std::max<uint32_t>(1, std::min<uint32_t>(want, sh_cdiv(k, BK)));
    const uint32_t kps = sh_cdiv(sh_cdiv(k, s), BK) * BK;
    return {sh_cdiv(k, kps), kps};
}

// Estimated seconds of config i for an (M, N, K) problem cut into `splits` K ranges (as split_k launches them):
// the larger of
//  - throughput: rounds of tiles over the CUs at the config's sustained MFMA fraction (also returned alone
//    in *thr), and
//  - latency: no workgroup finishes before its start-up and epilogue plus its chain of BK slices, counted
//    once per round of tiles. Both costs grow with the tile area A (in units of 1024 outputs); fitted to
//    kernel traces on MI355X (256 x {256, 2304, 768} x {256, 768, 3072} and 1024^3): direct-to-LDS kernels
//    3.0 + 0.16 A us + (0.17 + 0.02 A) us per slice, the register-staged kernel 1.0 + 0.32 A us + (0.88 +
//    0.013 A) us per slice;
// plus, in both, the split-K partial traffic and the reduction launch. Small problems are latency-bound.
double est_time(int i, uint32_t M, uint32_t N, uint32_t K, uint32_t want_splits, int cus, double *thr = nullptr) {
    const KCfg &c = g_cfgs[i];
    const SplitK sk = split_k(K, want_splits);
    const uint32_t splits = sk.splits;
    const double tiles = (double)sh_cdiv(M, c.bm) * sh_cdiv(N, c.bn) * splits;
    const double rounds = std::ceil(tiles / cus);
    const double k_len = (double)sk.kps;
    double t = rounds * c.bm * c.bn * k_len / (c.eff * 2048.0 * 2.4e9);
    const double A = c.bm * c.bn / 1024.0;
    const double fixed_us = c.v2 ? 3.0 + 0.16 * A : 1.0 + 0.32 * A;
    const double slice_us = c.v2 ? 0.17 + 0.02 * A : 0.88 + 0.013 * A;
    const double lat = 1e-6 * (fixed_us + rounds * (k_len / BK) * slice_us);
    const double split_cost = splits > 1 ? ((double)splits * M * N * 8.0 + (double)M * N * 2.0) / 5e12 + 4e-6 : 0.0;
    if (thr) *thr = t + split_cost;
    return std::max(t, lat) + split_cost;
}

struct Plan { int cfg; uint32_t splits; };

// fast: vector operands and K % 64 == 0; ktail: vector operands with a partial last k-slice
// A W^T call with aligned operands and K % 64 == 0 runs only on the W^T direct-to-LDS tiles, which store the bits
// of the W-layout direct-to-LDS tiles; otherwise it takes the register-staged tiles (the bits of the W-layout
// register-staged tiles).
bool eligible(const KCfg &c, bool vec, bool fast, bool ktail, bool wt, bool reg_only = false) {
    if (reg_only && !c.reg) return false;
    if (c.v2) return c.wt == wt && (fast || (!wt && ktail && c.ktail));
    if (wt && fast) return false;
    return vec || c.bm * c.bn <= 128 * 128;
}

// reg_only: only configurations whose unsplit epilogue applies a LayerNorm fold and writes row partials; if none is
// eligible the plan falls back to the unrestricted choice and the launch goes through the partials path.
Plan choose(uint32_t M, uint32_t N, uint32_t K, bool vec, bool fast, uint32_t want_splits, bool wt = false, bool reg_only = false) {
    const bool ktail = vec && K > 0 && K % BK != 0;
    const int cus = sh_num_cus() > 0 ? sh_num_cus() : 256;
    // Every eligible (config, splits) is estimated; among those within 3 % of the fastest estimate the one with
    // the lowest throughput term wins (tiles of one size share one latency floor; the throughput term ranks
    // them), the earlier config and fewer splits on a tie.
    struct Cand { double t, thr; int cfg; uint32_t splits; };
    Cand cand[kNumCfg * 16];
    int n = 0;
    double tmin = 1e300;
    for (int i = 0; i < kNumCfg; ++i) {
        if (!eligible(g_cfgs[i], vec, fast, ktail, wt, reg_only)) continue;
        uint32_t lo = 1, hi = 1;
        if (want_splits) lo = hi = want_splits;
        else hi = std::max<uint32_t>(1, std::min<uint32_t>(16, K / 128));
        uint32_t prev = 0;
        for (uint32_t s = lo; s <= hi && n < kNumCfg * 16; ++s) {
            const uint32_t eff = split_k(K, s).splits;          // requests that launch the same ranges count once
            if (eff == prev) continue;
            prev = eff;
            double thr = 0.0;
            const double tt = est_time(i, M, N, K, eff, cus, &thr);
            cand[n++] = {tt, thr, i, eff};
            tmin = std::min(tmin, tt);
        }
    }
    Plan best{4, 1};
    double bthr = 1e300;
    for (int j = 0; j < n; ++j)
        if (cand[j].t <= tmin * 1.03 && cand[j].thr < bthr) { bthr = cand[j].thr; best = {cand[j].cfg, cand[j].splits}; }
    const int fc = env_int("SH_GEMM_CFG", -1);
    const int fs = env_int("SH_GEMM_SPLITS", 0);
    if (fs > 0 && !want_splits) best.splits = split_k(K, (uint32_t)fs).splits;
    if (fc >= 0 && fc < kNumCfg && eligible(g_cfgs[fc], vec, fast, ktail, wt, reg_only)) best.cfg = fc;
    if (reg_only && n == 0) return choose(M, N, K, vec, fast, want_splits, wt, false);
    return best;
}

void set_attrs(KCfg &c) {
    if (c.attr_set) return;
    for (int v = 0; v < 2; ++v) {
        if (c.vec[v]) (void)hipFuncSetAttribute((const void *)c.vec[v], hipFuncAttributeMaxDynamicSharedMemorySize, (int)c.lds);
        if (c.scalar[v]) (void)hipFuncSetAttribute((const void *)c.scalar[v], hipFuncAttributeMaxDynamicSharedMemorySize, (int)c.lds);
        if (c.tail[v]) (void)hipFuncSetAttribute((const void *)c.tail[v], hipFuncAttributeMaxDynamicSharedMemorySize, (int)c.lds);
        if (c.wt_vec[v]) (void)hipFuncSetAttribute((const void *)c.wt_vec[v], hipFuncAttributeMaxDynamicSharedMemorySize, (int)c.lds);
        if (c.wt_scalar[v]) (void)hipFuncSetAttribute((const void *)c.wt_scalar[v], hipFuncAttributeMaxDynamicSharedMemorySize, (int)c.lds);
    }
    if (c.kg2) (void)hipFuncSetAttribute((const void *)c.kg2, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(2 * c.lds));
    for (int k = 1; k < EPI_KINDS; ++k)
        if (c.epi[k]) (void)hipFuncSetAttribute((const void *)c.epi[k], hipFuncAttributeMaxDynamicSharedMemorySize, (int)c.lds);
    c.attr_set = true;
}

// Workgroups of a launch (tiles_m, tiles_n and splits set): one per tile and K range; sets the XCD remap.
uint32_t grid_of(GemmArgs &a) {
    const uint32_t nblk = a.tiles_m * a.tiles_n * a.splits;
    const int X = sh_num_xcds();
    a.xcd_groups = (X > 1 && nblk % (uint32_t)X == 0) ? (uint32_t)X : 1;
    // bands of 8 tile rows: an XCD's 64 first tiles of a 128x192 tiling span 8 row panels and 8 column panels
    // (3.9 MB of operands at K = 768, inside its 4 MB L2) instead of 4 and every one (SH_GEMM_GROUP=1: row-major)
    static const int gm = env_int("SH_GEMM_GROUP", 8);
    a.group_m = gm > 1 ? (uint32_t)gm : 1;
    return nblk;
}

void set_grid(GemmArgs &a, const KCfg &c) {
    a.tiles_m = sh_cdiv(a.M, c.bm); a.tiles_n = sh_cdiv(a.N, c.bn);
}

// One-time timing of the tile configurations for a large unsplit problem. Every unsplit configuration
// accumulates K in the same order with the same MFMA, so they store bit-identical results and the choice only
// changes speed. Trial runs write a scratch output (no accumulate; bias, activation, residual, LayerNorm fold and
// row partials as in the call: the residual and fold rows are only read, the row partials are written again by
// the call itself); the winner is cached per shape and epilogue. Skipped under stream capture, for small
// problems, or SH_GEMM_TUNE=0.
typedef std::tuple<uint32_t, uint32_t, uint32_t, uint64_t, uint64_t, uint32_t, uint32_t, uint32_t> TuneKey;   // + flags
std::map<TuneKey, int> g_tuned;

// SH_GEMM_TUNE_FILE=path: choices are read from that file at the first tuning decision and every new choice is
// appended to it ("M N K ldx ldw bias act flags cfg" per line; flags: 1 W^T, 2 LayerNorm fold or row partials,
// 4 residual), so a later process (a counter run, under which the timing itself would be distorted) launches
// exactly the tiles an earlier timed run chose.
void tune_file_load() {
    static bool done = false;
    if (done) return;
    done = true;
    const char *path = getenv("SH_GEMM_TUNE_FILE");
    if (!path || !*path) return;
    FILE *f = fopen(path, "r");
    if (!f) return;
    unsigned M, N, K, b, act, wt; unsigned long long ldx, ldw; int cfg;
    while (fscanf(f, "%u %u %u %llu %llu %u %u %u %d", &M, &N, &K, &ldx, &ldw, &b, &act, &wt, &cfg) == 9)
        if (cfg >= 0 && cfg < kNumCfg && g_cfgs[cfg].v2 && g_cfgs[cfg].wt == ((wt & 1u) != 0) && (!(wt & 2u) || g_cfgs[cfg].reg))
            g_tuned[TuneKey{M, N, K, ldx, ldw, b, act, wt}] = cfg;
    fclose(f);
}

void tune_file_append(const TuneKey &k, int cfg) {
    const char *path = getenv("SH_GEMM_TUNE_FILE");
    if (!path || !*path) return;
    FILE *f = fopen(path, "a");
    if (!f) return;
    fprintf(f, "%u %u %u %llu %llu %u %u %u %d\n", std::get<0>(k), std::get<1>(k), std::get<2>(k), (unsigned long long)std::get<3>(k),
            (unsigned long long)std::get<4>(k), std::get<5>(k), std::get<6>(k), std::get<7>(k), cfg);
    fclose(f);
}

// The k_gemm5 epilogue build (EPI) for an unsplit call's epilogue, or 0 for the build that reads every flag:
// the LayerNorm fold with its fp32 d row and GELU or nothing after it; fp16 bias + residual + row partials; fp16
// bias alone, with GELU after it, or with a residual; none. SH_GEMM_EPI=0 keeps every call on the general build
// (tests compare the two).
int gemm_epi_kind(const GemmArgs &a) {
    if (a.accumulate || env_int("SH_GEMM_EPI", 1) == 0) return EPI_ANY;
    if (!a.bias) return !a.ln_stats && !a.res && !a.stats_out && a.act == SH_ACT_NONE ? EPI_PLAIN : EPI_ANY;
    if (a.ln_stats && a.bias_fp32 && !a.res && !a.stats_out)
        return a.act == SH_ACT_GELU ? EPI_FOLD_GELU : a.act == SH_ACT_NONE ? EPI_FOLD : EPI_ANY;
    if (a.ln_stats || a.bias_fp32) return EPI_ANY;
    if (a.res && a.stats_out) return a.act == SH_ACT_NONE ? EPI_BIAS_RES_STATS : EPI_ANY;
    if (a.stats_out) return EPI_ANY;
    if (a.res) return a.act == SH_ACT_NONE ? EPI_BIAS_RES : EPI_ANY;
    return a.act == SH_ACT_GELU ? EPI_BIAS_GELU : a.act == SH_ACT_NONE ? EPI_BIAS : EPI_ANY;
}
// The kernel an unsplit, vector-path call of tile configuration c launches.
KernelFn unsplit_kernel(const KCfg &c, const GemmArgs &a) {
    const int ek = gemm_epi_kind(a);
    // (the epilogue builds address Z, the residual and their operand DMAs with 32-bit byte offsets from scalar bases)
    const bool off32 = ((uint64_t)a.M * a.ldz + a.N) * 2 < (1ull << 32) && (!a.res || ((uint64_t)a.M * a.ldr + a.N) * 2 < (1ull << 32)) &&
                       a.M < (1u << 24) && a.N < (1u << 24) && a.ldz < (1u << 24) && a.ldr < (1u << 24) && a.ldx < (1u << 22) &&
                       a.ldw < (1u << 22) && (uint64_t)a.M * a.N / 4 < (1ull << 32);
    return ek != EPI_ANY && c.epi[ek] && off32 ? c.epi[ek] : c.vec[0];
}

int tuned_cfg(const GemmArgs &call, int heur, hipStream_t st, bool wt) {
    const bool reg_only = call.ln_stats != nullptr || call.stats_out != nullptr;
    static const int enabled = env_int("SH_GEMM_TUNE", 1);
    if (!enabled || env_int("SH_GEMM_CFG", -1) >= 0) return heur;
    const int cus = sh_num_cus() > 0 ? sh_num_cus() : 256;
    double thr = 0.0;
    (void)est_time(heur, call.M, call.N, call.K, 1, cus, &thr);
    if (thr < 6e-6) return heur;                     // the throughput estimate: small problems keep the model's tile
    tune_file_load();
    const TuneKey key{call.M, call.N, call.K, call.ldx, call.ldw, call.bias ? 1u + call.bias_fp32 : 0u, call.act,
                      (wt ? 1u : 0u) | (reg_only ? 2u : 0u) | (call.res ? 4u : 0u)};
    auto it = g_tuned.find(key);
    if (it != g_tuned.end()) return it->second;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return heur;
    uint16_t *scratch = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipMalloc(&scratch, (size_t)call.M * call.N * 2) != hipSuccess) { (void)hipGetLastError(); return heur; }
    int best = heur;
    if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        GemmArgs a = call;
        a.z = scratch; a.ldz = call.N; a.accumulate = 0; a.splits = 1; a.part = nullptr;
        // three interleaved rounds, the minimum per configuration: one slow sample does not decide the choice
        float mins[kNumCfg];
        for (float &m : mins) m = 1e30f;
        bool ok = true;
        for (int round = 0; round < 3 && ok; ++round)
            for (int i = 0; i < kNumCfg && ok; ++i) {
                KCfg &c = g_cfgs[i];
                if (!c.v2 || c.wt != wt || (reg_only && !c.reg)) continue;
                set_attrs(c);
                set_grid(a, c);
                const dim3 grid(grid_of(a));
                const KernelFn kf = unsplit_kernel(c, a);     // (the build the call itself would launch)
                if (round == 0) hipLaunchKernelGGL(kf, grid, dim3(c.threads), c.lds, st, a);     // warm-up
                (void)hipEventRecord(e0, st);
                for (int rep = 0; rep < 2; ++rep) hipLaunchKernelGGL(kf, grid, dim3(c.threads), c.lds, st, a);
                (void)hipEventRecord(e1, st);
                float ms = 0.f;
                ok = hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
                if (ok && ms < mins[i]) mins[i] = ms;
            }
        if (ok) {
            float best_ms = 1e30f;
            for (int i = 0; i < kNumCfg; ++i)
                if (g_cfgs[i].v2 && g_cfgs[i].wt == wt && (!reg_only || g_cfgs[i].reg) && mins[i] < best_ms) { best_ms = mins[i]; best = i; }
            if (env_int("SH_GEMM_VERBOSE", 0)) {      // the one-time choice on stderr: model pick, winner, all times
                fprintf(stderr, "[sh_gemm] tuned %ux%ux%u: model cfg %d (%.2f us), chose cfg %d (%.2f us);", call.M, call.N, call.K,
                        heur, 500.f * mins[heur], best, 500.f * best_ms);
                for (int i = 0; i < kNumCfg; ++i)
                    if (g_cfgs[i].v2 && g_cfgs[i].wt == wt && (!reg_only || g_cfgs[i].reg)) fprintf(stderr, " %d:%.2f", i, 500.f * mins[i]);
                fprintf(stderr, "\n");
            }
        }
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(st);
    (void)hipFree(scratch);
    (void)hipGetLastError();
    g_tuned[key] = best;
    tune_file_append(key, best);
    return best;
}

struct GemmReq {
    uint64_t x, w, z; uint32_t M, N, K; uint32_t ldx, ldw, ldz;
    uint32_t accumulate; const sh_gemm_epi *epi; uint32_t splits; bool mesh;
    float *part = nullptr;       // non-null: split-K partials go here (no workspace, no one-time tile timing)
    bool wt = false;             // w holds W^T ([N, K], leading dim ldw)
};

// Split-K partials of sh_gemm_splitk_noalloc: a fixed array in every GPU's copy of the code object, so that entry
// point allocates nothing. Its device address is looked up once per device (hipGetSymbolAddress with that device
// current); host code uses that address, never the array's name (which is only a host-side stand-in).
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
__device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];
std::map<int, float *> g_scratch_ptr;

float *scratch_ptr() {
    int dev = -1;
    if (!sh_hip_ok(hipGetDevice(&dev), "sh_gemm_splitk_noalloc hipGetDevice")) return nullptr;
    auto it = g_scratch_ptr.find(dev);
    if (it != g_scratch_ptr.end()) return it->second;
    void *p = nullptr;
    if (!sh_hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "sh_gemm_splitk_noalloc hipGetSymbolAddress")) return nullptr;
    if (!p) { sh_set_error(SH_EHIP, "[sh_gemm_splitk_noalloc] scratch array has no device address"); return nullptr; }
    g_scratch_ptr[dev] = (float *)p;
    return (float *)p;
}

int launch(const GemmReq &r, const char *name) {
    if (r.M == 0 || r.N == 0) return 0;
    const sh_gemm_epi *e = r.epi;
    const uint64_t bias = e ? e->bias : 0, res = e ? e->residual : 0;
    const uint32_t ldr = e ? e->ldr : 0;
    const bool vec = r.N % 8 == 0 && r.K % 8 == 0 && r.ldx % 8 == 0 && r.ldw % 8 == 0 && r.ldz % 8 == 0 &&
                     sh_aligned16(r.x) && sh_aligned16(r.w) && sh_aligned16(r.z) &&
                     (!res || (ldr % 8 == 0 && sh_aligned16(res))) && (!bias || sh_aligned16(bias));
    const bool fast = vec && r.K % BK == 0 && r.K > 0;
    // LayerNorm fold and row partials: the unsplit kernels that apply the fold on their fp32 accumulators (16-byte
    // aligned c / d rows) and write the partials from their registers; every other case goes through the fp32
    // partials (one K range or more) and the reduction does both
    const bool ln = e && e->ln_stats;
    const bool stats = e && e->stats_out;
    if (stats && (!vec || r.N % 32 != 0)) {
        sh_set_error(-1, "[%s] row partials need N %% 32 == 0 and 16-byte aligned operands and leading dims", name);
        return -1;
    }
    const bool ln_reg = ln && fast && sh_aligned16(e->ln_c) && sh_aligned16(bias);
    const bool want_reg = (ln || stats) && fast && (!ln || ln_reg);
    Plan p = choose(r.M, r.N, r.K, vec, fast, r.splits, r.wt, want_reg);
    if (r.mesh) p.splits = 1;
    auto set_epi = [&](GemmArgs &t) {
        t.ln_stats = ln ? (const float *)e->ln_stats : nullptr; t.ln_c = ln ? (const float *)e->ln_c : nullptr;
        t.ln_parts = ln ? e->ln_parts : 0; t.ln_eps = ln ? e->ln_eps : 0.f;
        t.stats_out = stats ? (float *)e->stats_out : nullptr;
    };
    if (fast && p.splits == 1 && g_cfgs[p.cfg].v2 && !r.part && (!(ln || stats) || (want_reg && g_cfgs[p.cfg].reg))) {
        GemmArgs t{};
        t.x = (const uint16_t *)r.x; t.w = (const uint16_t *)r.w; t.bias = (const void *)bias;
        t.ldx = r.ldx; t.ldw = r.ldw; t.M = r.M; t.N = r.N; t.K = r.K; t.kps = sh_cdiv(r.K, BK) * BK; t.splits = 1;
        t.bias_fp32 = (e && e->bias_fmt == SH_BIAS_FP32) ? 1 : 0; t.act = e ? e->act : 0;
        t.res = (const uint16_t *)res; t.ldr = ldr;
        set_epi(t);
        p.cfg = tuned_cfg(t, p.cfg, sh_stream(), r.wt);
    }
    const SplitK sk = split_k(r.K, p.splits);
    const uint32_t splits = sk.splits, kps = sk.kps;
    // Two equal K ranges (a caller's request for 2 splits, K % 128 == 0) planned on a direct-to-LDS tile run
    // in-workgroup (k_gemm5 KG = 2): that family's bits for two partials and the reduction, without either (the
    // register-staged tiles accumulate in another order). The planned tile if it has the variant, else the first
    // that has. SH_GEMM_KG=0: the partials path (tests compare the two).
    int kgc = -1;
    if (fast && !r.wt && splits == 2 && 2 * kps == r.K && g_cfgs[p.cfg].v2 && (!(ln || stats) || want_reg) &&
        env_int("SH_GEMM_KG", 1)) {
        for (int i = 0; i < kNumCfg && kgc < 0; ++i)
            if (g_cfgs[i].kg2) kgc = i;
        if (g_cfgs[p.cfg].kg2) kgc = p.cfg;
    }
    const bool kg2 = kgc >= 0;
    KCfg &c = g_cfgs[kg2 ? kgc : p.cfg];
    const bool partials = !kg2 && (splits > 1 || ((ln || stats) && !(want_reg && c.reg)));

    GemmArgs a{};
    a.x = (const uint16_t *)r.x; a.w = (const uint16_t *)r.w; a.z = (uint16_t *)r.z;
    a.bias = (const void *)bias; a.res = (const uint16_t *)res;
    a.ldx = r.ldx; a.ldw = r.ldw; a.ldz = r.ldz; a.ldr = ldr;
    a.M = r.M; a.N = r.N; a.K = r.K; a.kps = kps;
    a.tiles_m = sh_cdiv(r.M, c.bm); a.tiles_n = sh_cdiv(r.N, c.bn); a.splits = kg2 ? 1 : splits;
    a.accumulate = r.accumulate; a.bias_fp32 = (e && e->bias_fmt == SH_BIAS_FP32) ? 1 : 0; a.act = e ? e->act : 0;
    set_epi(a);
    const uint64_t nblk64 = (uint64_t)a.tiles_m * a.tiles_n * a.splits;
    if (nblk64 > 0x7FFFFFFFull) { sh_set_error(-1, "[%s] problem too large", name); return -1; }
    const uint32_t nblk = grid_of(a);

    hipStream_t st = sh_stream();
    const bool split = partials;
    KernelFn fn = kg2 ? c.kg2
                : r.wt ? (c.v2 ? c.vec[split] : vec ? c.wt_vec[split] : c.wt_scalar[split])
                       : (c.v2 && !fast) ? c.tail[split] : (vec || c.v2) ? c.vec[split] : c.scalar[split];   // !fast: K % 64 != 0
    if (!kg2 && !split && !r.wt && fast && c.v2) fn = unsplit_kernel(c, a);
    set_attrs(c);
    if (split) {
        const size_t ws = (size_t)splits * r.M * r.N * sizeof(float);
        if (r.part) {
            if (ws > kNoAllocScratchBytes) {
                sh_set_error(-1, "[%s] %u splits of %ux%u fp32 partials need %zu B > the %zu B scratch", name, splits, r.M, r.N,
                             ws, kNoAllocScratchBytes);
                return -1;
            }
            a.part = r.part;
        } else {
            a.part = (float *)sh_workspace(ws);
            if (!a.part) return SH_EHIP;
        }
    }
    hipLaunchKernelGGL(fn, dim3(nblk), dim3(kg2 ? 2 * c.threads : c.threads), kg2 ? 2 * c.lds : c.lds, st, a);
    if (!sh_launch_ok(name)) return SH_EHIP;
    if (split) {
        const bool rvec = vec;
        const uint32_t per_row = rvec ? r.N / 8 : r.N;
        const uint64_t items = (uint64_t)r.M * per_row;
        if (items > 0xFFFFFF00ull) { sh_set_error(-1, "[%s] problem too large", name); return -1; }
        const ShDiv div = sh_make_div(per_row);
        if (rvec) hipLaunchKernelGGL(k_splitk_reduce<true>, dim3(sh_cdiv((uint32_t)items, 64)), dim3(64), 0, st, a, div, per_row, (uint32_t)items);
        else hipLaunchKernelGGL(k_splitk_reduce<false>, dim3(sh_cdiv((uint32_t)items, 64)), dim3(64), 0, st, a, div, per_row, (uint32_t)items);
        if (!sh_launch_ok(name)) return SH_EHIP;
    }
    return 0;
}

// The LayerNorm fold's arguments: both rows given, the bias is the fp32 row d, and no accumulate (z_old would
// be added after the fold's rounding point, which no unfused sequence does); partial statistics cover the K
// columns the fold normalises. Row partials go to an 8-byte aligned [M][N / 32] pair array.
int check_ln(const char *name, const sh_gemm_epi *e, const sh_gemm_cfg &c, uint32_t K) {
    if (e && e->stats_out % 8) { sh_set_error(-1, "[%s] stats_out must be 8-byte aligned", name); return -1; }
    if (!e || (!e->ln_stats && !e->ln_c)) return 0;
    if (!e->ln_stats || !e->ln_c || !e->bias || e->bias_fmt != SH_BIAS_FP32 || c.accumulate) {
        sh_set_error(-1, "[%s] LayerNorm fold needs ln_stats, ln_c and the fp32 bias row d, without accumulate", name);
        return -1;
    }
    if ((e->ln_c | e->bias) % 4) { sh_set_error(-1, "[%s] LayerNorm fold rows must be 4-byte aligned", name); return -1; }
    if (e->ln_stats % 8) { sh_set_error(-1, "[%s] ln_stats ((mu, r) or partial pairs) must be 8-byte aligned", name); return -1; }
    if (e->ln_parts && (uint64_t)e->ln_parts * 32 != K) {
        sh_set_error(-1, "[%s] %u row partials of 32 columns do not cover K = %u", name, e->ln_parts, K);
        return -1;
    }
    if (e->ln_parts && !(e->ln_eps >= 0.f)) { sh_set_error(-1, "[%s] ln_eps must be >= 0", name); return -1; }
    return 0;
}

void cfg_fill(sh_gemm_cfg *c, const sh_gemm_cfg *in) {   // sh_gemm.inc.c:17-22
    if (in) *c = *in;
    else { c->tm = c->tn = c->tk = 0; c->pipeline = 1; c->accumulate = 0; c->fmt = 0; c->l1_base = 0; }
    if (!c->tm) c->tm = 256;
    if (!c->tn) c->tn = 256;
    if (!c->tk) c->tk = 256;
}

// The reference's checks (sh_gemm.inc.c:60-68): -1 tile divisibility, -2 TCDM budget; plus fmt / NULL.
int check_tiled(const char *name, const sh_gemm_cfg &c, uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K) {
    if (M % c.tm || N % c.tn || K % c.tk) {
        sh_set_error(-1, "[%s] shape %ux%ux%u not divisible by tile %ux%ux%u", name, M, N, K, c.tm, c.tn, c.tk);
        return -1;
    }
    const uint32_t need = sh_gemm_l1_bytes(M, N, K, &c);
    if (need > SH_REF_TCDM_BYTES) {
        sh_set_error(-2, "[%s] L1 need %u > %u", name, need, SH_REF_TCDM_BYTES);
        return -2;
    }
    if (c.fmt != SH_FP16) { sh_set_error(-1, "[%s] fmt %u: only SH_FP16 is implemented", name, c.fmt); return -1; }
    if (!x || !w || !z) { sh_set_error(-1, "[%s] NULL tensor address", name); return -1; }
    return 0;
}

}  // namespace

extern "C" {

uint32_t sh_gemm_l1_bytes(uint32_t, uint32_t, uint32_t, const sh_gemm_cfg *cfg) {
    sh_gemm_cfg c;
    cfg_fill(&c, cfg);
    const uint32_t xb = c.tm * c.tk * 2, wb = c.tk * c.tn * 2, yb = c.tm * c.tn * 2;   // uint32 as in the reference
    const uint32_t nbuf = c.pipeline ? 2 : 1;
    return c.l1_base + nbuf * (xb + wb) + yb;
}

int sh_gemm(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
            uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, uint32_t) {
    sh_gemm_cfg c;
    cfg_fill(&c, cfg);
    if (int rc = check_tiled("sh_gemm", c, x, w, z, M, N, K)) return rc;
    GemmReq r{x, w, z, M, N, K, ldx, ldw, ldz, c.accumulate, nullptr, 1, false};
    return launch(r, "sh_gemm");
}

int sh_gemm_splitk(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                   uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, uint32_t splits, uint32_t) {
    sh_gemm_cfg c;
    cfg_fill(&c, cfg);
    if (int rc = check_tiled("sh_gemm_splitk", c, x, w, z, M, N, K)) return rc;
    GemmReq r{x, w, z, M, N, K, ldx, ldw, ldz, c.accumulate, nullptr, splits, false};
    return launch(r, "sh_gemm_splitk");
}

// sh_gemm_splitk with the partials in the library's fixed scratch array: no hipMalloc / hipFree and no one-time
// tile timing (that allocates a trial output). A launch that writes fp32 partials must need at most 16 MiB of them
// (splits x M x N x 4 bytes), else -1 before any GPU work (launch() checks it on that path only: two equal K ranges
// of a direct-to-LDS plan run in one workgroup and write no partials). Every call on one GPU shares its array:
// calls that overlap on one GPU (different streams, or host threads) race on it. Each call writes every partial
// it reads, so nothing has to be cleared between calls.
int sh_gemm_splitk_noalloc(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                           uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, uint32_t splits, uint32_t) {
    sh_gemm_cfg c;
    cfg_fill(&c, cfg);
    if (int rc = check_tiled("sh_gemm_splitk_noalloc", c, x, w, z, M, N, K)) return rc;
    sh_ensure_init();
    float *part = scratch_ptr();
    if (!part) return SH_EHIP;
    GemmReq r{x, w, z, M, N, K, ldx, ldw, ldz, c.accumulate, nullptr, splits, false, part};
    return launch(r, "sh_gemm_splitk_noalloc");
}

int sh_gemm_tile_count(void) { return kNumCfg; }

int sh_gemm_tile_info(uint32_t i, uint32_t *out) {
    if (i >= (uint32_t)kNumCfg || !out) { sh_set_error(-1, "[sh_gemm_tile_info] no configuration %u or NULL output", i); return -1; }
    const KCfg &c = g_cfgs[i];
    out[0] = (uint32_t)c.bm; out[1] = (uint32_t)c.bn;
    out[2] = !c.v2 ? 1u : c.wt ? 6u : c.ktail ? 2u : 5u;
    out[3] = (uint32_t)c.threads; out[4] = c.wt; out[5] = c.reg; out[6] = c.kg2 != nullptr; out[7] = c.ktail;
    return 0;
}

// The cost model's plan for 16-byte-aligned operands (what a call would launch before the one-time timing of a
// large problem): out = {tile configuration, tile rows, tile columns, split count}. No GPU work; 256 CUs are
// assumed when no GPU is visible. SH_GEMM_CFG / SH_GEMM_SPLITS apply as for a call.
int sh_gemm_plan(uint32_t M, uint32_t N, uint32_t K, uint32_t splits, uint32_t *out) {
    if (!M || !N || !K || !out) { sh_set_error(-1, "[sh_gemm_plan] empty problem or NULL output"); return -1; }
    const bool vec = N % 8 == 0 && K % 8 == 0;
    const Plan p = choose(M, N, K, vec, vec && K % BK == 0, splits);
    out[0] = (uint32_t)p.cfg;
    out[1] = (uint32_t)g_cfgs[p.cfg].bm;
    out[2] = (uint32_t)g_cfgs[p.cfg].bn;
    out[3] = p.splits;
    return 0;
}

int sh_gemm_ex(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
               uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, const sh_gemm_epi *epi) {
    sh_gemm_cfg c;
    cfg_fill(&c, cfg);
    if (!x || !w || !z) { sh_set_error(-1, "[sh_gemm_ex] NULL tensor address"); return -1; }
    if (c.fmt != SH_FP16) { sh_set_error(-1, "[sh_gemm_ex] fmt %u: only SH_FP16 is implemented", c.fmt); return -1; }
    if (epi && epi->residual && epi->ldr < N) { sh_set_error(-1, "[sh_gemm_ex] ldr %u < N %u", epi->ldr, N); return -1; }
    if (epi && epi->act > SH_ACT_GELU) { sh_set_error(-1, "[sh_gemm_ex] unknown act %u", epi->act); return -1; }
    if (int rc = check_ln("sh_gemm_ex", epi, c, K)) return rc;
    GemmReq r{x, w, z, M, N, K, ldx, ldw, ldz, c.accumulate, epi, epi ? epi->splits : 1u, false};
    return launch(r, "sh_gemm_ex");
}

int sh_gemm_ex_wt(uint64_t x, uint64_t wt, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                  uint32_t ldx, uint32_t ldwt, uint32_t ldz, const sh_gemm_cfg *cfg, const sh_gemm_epi *epi) {
    sh_gemm_cfg c;
    cfg_fill(&c, cfg);
    if (!x || !wt || !z) { sh_set_error(-1, "[sh_gemm_ex_wt] NULL tensor address"); return -1; }
    if (c.fmt != SH_FP16) { sh_set_error(-1, "[sh_gemm_ex_wt] fmt %u: only SH_FP16 is implemented", c.fmt); return -1; }
    if (ldwt < K) { sh_set_error(-1, "[sh_gemm_ex_wt] ldwt %u < K %u", ldwt, K); return -1; }
    if (epi && epi->residual && epi->ldr < N) { sh_set_error(-1, "[sh_gemm_ex_wt] ldr %u < N %u", epi->ldr, N); return -1; }
    if (epi && epi->act > SH_ACT_GELU) { sh_set_error(-1, "[sh_gemm_ex_wt] unknown act %u", epi->act); return -1; }
    if (int rc = check_ln("sh_gemm_ex_wt", epi, c, K)) return rc;
    GemmReq r{x, wt, z, M, N, K, ldx, ldwt, ldz, c.accumulate, epi, epi ? epi->splits : 1u, false};
    r.wt = true;
    return launch(r, "sh_gemm_ex_wt");
}

int sh_gemm_mesh(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                 uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg) {
    sh_gemm_cfg c;
    cfg_fill(&c, cfg);
    const uint32_t P = SH_MESH_P, T = c.tm;
    if (c.tn != T || M != P * T || N != P * T || K % c.tk) {       // sh_gemm.inc.c:134-138
        sh_set_error(-1, "[sh_gemm_mesh] need square mesh, tm==tn, M==N==P*tm, K%%tk==0 (got %ux%ux%u tile %ux%ux%u mesh %ux%u)",
                     M, N, K, c.tm, c.tn, c.tk, P, P);
        return -1;
    }
    if (sh_gemm_l1_bytes(M, N, K, &c) > SH_REF_TCDM_BYTES) {      // sh_gemm.inc.c:139-142
        sh_set_error(-2, "[sh_gemm_mesh] L1 budget exceeded");
        return -2;
    }
    if (c.fmt != SH_FP16) { sh_set_error(-1, "[sh_gemm_mesh] fmt %u: only SH_FP16 is implemented", c.fmt); return -1; }
    if (!x || !w || !z) { sh_set_error(-1, "[sh_gemm_mesh] NULL tensor address"); return -1; }
    GemmReq r{x, w, z, M, N, K, ldx, ldw, ldz, c.accumulate, nullptr, 1, true};
    return launch(r, "sh_gemm_mesh");
}

}  // extern "C"

// ---- small-M GEMM (reference sh_gemm.inc.c:192-344) ----------------------------------------------------------
// The reference streams each cluster's W column slice while X is multicast once over its mesh. On the GPU X (M <= a
// few hundred rows) is re-read from L2 by every column tile and W crosses HBM once, so the work is the tiled GEMM
// with a split count chosen for the few output tiles of a small M. The plan (column slice per cluster, K panel,
// whole / panel schedule) and its TCDM bytes are computed exactly as the reference computes them, on its 16-cluster
// mesh, so sh_gemm_xmcast_l1_bytes and the -1 / -2 / -3 answers match.
namespace {
constexpr uint32_t kXmClusters = 16;          // ARCH_NUM_CLUSTER_X * ARCH_NUM_CLUSTER_Y of the reference mesh
constexpr uint32_t kXmL1Limit = 0x90000u;     // SH_XM_L1_LIMIT (sh_gemm.inc.c:210)
constexpr uint32_t kXmWholeMax = 0x50000u;    // SH_XM_WHOLE_MAX (sh_gemm.inc.c:214)

uint32_t xm_need(uint32_t rows, uint32_t K, uint32_t Nc, uint32_t tk, uint32_t whole) {   // sh_gemm.inc.c:219-221
    return (whole ? rows * K * 2 : 2 * rows * tk * 2) + 2 * tk * Nc * 2 + rows * Nc * 2;
}

// 0 and *end = the scratch end offset, or a negative reason (sh_gemm.inc.c:223-251)
int xm_plan(uint32_t M, uint32_t N, uint32_t K, const sh_gemm_cfg &c, uint32_t mode, uint32_t *end) {
    const uint32_t g = c.tn ? c.tn : 4;
    const uint32_t rows = c.tm ? c.tm : M;
    if (rows == 0 || M % rows) return -1;
    const uint32_t Nc = ((N + kXmClusters - 1) / kXmClusters + g - 1) / g * g;
    if (c.l1_base >= kXmL1Limit) return -2;
    const uint32_t lim = kXmL1Limit - c.l1_base;
    const bool try_whole = mode == SH_XM_WHOLE || (mode == SH_XM_AUTO && rows * K * 2 <= kXmWholeMax);
    for (int w = try_whole ? 1 : 0; w >= 0; --w) {
        if (mode == SH_XM_WHOLE && !w) break;
        uint32_t tk = 0;
        if (c.tk) {
            if (K % c.tk == 0 && xm_need(rows, K, Nc, c.tk, (uint32_t)w) <= lim) tk = c.tk;
        } else {
            for (uint32_t d = K < 256 ? K : 256; d; --d)
                if (K % d == 0 && xm_need(rows, K, Nc, d, (uint32_t)w) <= lim) { tk = d; break; }
        }
        if (!tk) continue;
        *end = c.l1_base + xm_need(rows, K, Nc, tk, (uint32_t)w);
        return 0;
    }
    return -2;
}

void xm_cfg(sh_gemm_cfg *c, const sh_gemm_cfg *in) {   // fields 0 mean "auto" here (sh_gemm.inc.c:261)
    if (in) *c = *in;
    else { c->tm = c->tn = c->tk = 0; c->pipeline = 1; c->accumulate = 0; c->fmt = 0; c->l1_base = 0; }
}
}  // namespace

extern "C" {

uint32_t sh_gemm_xmcast_l1_bytes(uint32_t M, uint32_t N, uint32_t K, const sh_gemm_cfg *cfg, uint32_t mode) {
    sh_gemm_cfg c;
    xm_cfg(&c, cfg);
    uint32_t end = 0;
    return xm_plan(M, N, K, c, mode, &end) ? 0xFFFFFFFFu : end;
}

int sh_gemm_xmcast_ex(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                      uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, uint32_t mode) {
    sh_gemm_cfg c;
    xm_cfg(&c, cfg);
    uint32_t end = 0;
    const int rc = (c.fmt & 3) ? -3 : xm_plan(M, N, K, c, mode, &end);
    if (rc) {
        sh_set_error(rc, "[sh_gemm_xmcast] %ux%ux%u tile %u,%u,%u mode %u: no plan (%d)", M, N, K, c.tm, c.tn, c.tk, mode, rc);
        return rc;
    }
    if (!x || !w || !z) { sh_set_error(-1, "[sh_gemm_xmcast] NULL tensor address"); return -1; }
    GemmReq r{x, w, z, M, N, K, ldx, ldw, ldz, c.accumulate, nullptr, 0, false};
    return launch(r, "sh_gemm_xmcast");
}

int sh_gemm_xmcast(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                   uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg) {
    return sh_gemm_xmcast_ex(x, w, z, M, N, K, ldx, ldw, ldz, cfg, SH_XM_AUTO);
}

}  // extern "C"

