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
#include <cstdlib>
#include <cstring>

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
};

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

template <int BM, int BN, bool VEC, bool SPLIT>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
    using C = Cfg<BM, BN>;
    extern __shared__ uint4 smem[];
    uint4 *sA = smem;                       // [2][BM * 8]
    uint4 *sB = smem + 2 * BM * 8;          // [2][BN * 8]

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1, g = lane >> 5, r32 = lane & 31;

    // workgroup -> (split, tile_m, tile_n)
    const uint32_t nblk = a.tiles_m * a.tiles_n * a.splits;
    uint32_t L = blockIdx.x;
    if (a.xcd_groups > 1) L = (blockIdx.x % a.xcd_groups) * (nblk / a.xcd_groups) + blockIdx.x / a.xcd_groups;
    const uint32_t tn = L % a.tiles_n, rest = L / a.tiles_n;
    const uint32_t tm = rest % a.tiles_m, split = rest / a.tiles_m;
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

    auto gload = [&](int kt) {
        const uint32_t k0 = kbeg + (uint32_t)kt * BK;
#pragma unroll
        for (int i = 0; i < C::A_PER_T; ++i) {
            const int c = t + 256 * i, row = c >> 3, kc = c & 7;
            ra[i] = load8<VEC>(a.x, a.ldx, m0 + row, k0 + 8 * kc, a.M, kend);
        }
        if (bload) {
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
        if (bload) {
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

    // accumulator element (i, j, r) -> tile row wm*TM + 32 i + 8 (r/4) + 4 g + r%4, column wn*TN + 32 j + r32
    if (SPLIT) {
        float *P = a.part + (uint64_t)split * a.M * a.N;
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                const uint32_t gn = n0 + wn * C::TN + j * 32 + r32;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t gm = m0 + wm * C::TM + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (gm < a.M && gn < a.N) P[(uint64_t)gm * a.N + gn] = acc[i][j][r];
                }
            }
        return;
    }

    uint16_t *sC = (uint16_t *)smem;        // fp16 tile [BM][BN], 16-byte chunk c of row r at c ^ (r & 7)
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) {
            const uint32_t col = wn * C::TN + j * 32 + r32, gn = n0 + col;
            float bv = 0.f;
            if (a.bias && gn < a.N) bv = a.bias_fp32 ? ((const float *)a.bias)[gn] : sh_dev_h2f(((const uint16_t *)a.bias)[gn]);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = wm * C::TM + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3), gm = m0 + row;
                float v = acc[i][j][r];
                if (a.accumulate && gm < a.M && gn < a.N) v += sh_dev_h2f(a.z[(uint64_t)gm * a.ldz + gn]);
                v += bv;
                if (a.act == SH_ACT_GELU) v = sh_gelu_f(v);
                sC[row * BN + (((col >> 3) ^ (row & 7)) << 3) + (col & 7)] = sh_dev_f2h(v);
            }
        }
    __syncthreads();
    constexpr int CPR = BN / 8;             // 16-byte chunks per tile row
    for (int c = t; c < BM * CPR; c += 256) {
        const int row = c / CPR, ch = c % CPR;
        const uint32_t gm = m0 + row, gn = n0 + 8 * ch;
        if (gm >= a.M || gn >= a.N) continue;
        uint4 q = ((const uint4 *)sC)[row * CPR + (ch ^ (row & 7))];
        if (VEC) {
            if (a.res) {
                const uint4 rq = *(const uint4 *)(a.res + (uint64_t)gm * a.ldr + gn);
                uint32_t o[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const uint32_t u = comp(q, p), v = comp(rq, p);
                    const float lo = sh_dev_h2f((uint16_t)(u & 0xFFFF)) + sh_dev_h2f((uint16_t)(v & 0xFFFF));
                    const float hi = sh_dev_h2f((uint16_t)(u >> 16)) + sh_dev_h2f((uint16_t)(v >> 16));
                    o[p] = (uint32_t)sh_dev_f2h(lo) | ((uint32_t)sh_dev_f2h(hi) << 16);
                }
                q = make_uint4(o[0], o[1], o[2], o[3]);
            }
            *(uint4 *)(a.z + (uint64_t)gm * a.ldz + gn) = q;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (gn + e >= a.N) break;
                uint16_t h = (uint16_t)(comp(q, e >> 1) >> (16 * (e & 1)));
                if (a.res) h = sh_dev_f2h(sh_dev_h2f(h) + sh_dev_h2f(a.res[(uint64_t)gm * a.ldr + gn + e]));
                a.z[(uint64_t)gm * a.ldz + gn + e] = h;
            }
        }
    }
}

// Sum of the split partials in split order, then the epilogue of k_gemm. Item = 8 columns (VEC) or 1.
template <bool VEC>
__global__ __launch_bounds__(256) void k_splitk_reduce(GemmArgs a, ShDiv div, uint32_t per_row, uint32_t items) {
    const uint32_t it = blockIdx.x * 256u + threadIdx.x;
    if (it >= items) return;
    const uint32_t gm = sh_div(it, div), cc = it - gm * per_row;
    const uint64_t plane = (uint64_t)a.M * a.N;
    constexpr int W = VEC ? 8 : 1;
    const uint32_t gn = VEC ? 8 * cc : cc;
    float v[W];
#pragma unroll
    for (int e = 0; e < W; ++e) v[e] = 0.f;
    for (uint32_t s = 0; s < a.splits; ++s) {
        const float *p = a.part + s * plane + (uint64_t)gm * a.N + gn;
        if (VEC) {
            const float4 u0 = *(const float4 *)p, u1 = *(const float4 *)(p + 4);
            v[0] += u0.x; v[1] += u0.y; v[2] += u0.z; v[3] += u0.w;
            v[4 % W] += u1.x; v[5 % W] += u1.y; v[6 % W] += u1.z; v[7 % W] += u1.w;
        } else {
            v[0] += p[0];
        }
    }
    uint16_t out[W];
#pragma unroll
    for (int e = 0; e < W; ++e) {
        const uint32_t n = gn + e;
        float x = v[e];
        if (a.accumulate) x += sh_dev_h2f(a.z[(uint64_t)gm * a.ldz + n]);
        if (a.bias) x += a.bias_fp32 ? ((const float *)a.bias)[n] : sh_dev_h2f(((const uint16_t *)a.bias)[n]);
        if (a.act == SH_ACT_GELU) x = sh_gelu_f(x);
        uint16_t h = sh_dev_f2h(x);
        if (a.res) h = sh_dev_f2h(sh_dev_h2f(h) + sh_dev_h2f(a.res[(uint64_t)gm * a.ldr + n]));
        out[e] = h;
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
struct KCfg { int bm, bn; KernelFn vec[2], scalar[2]; size_t lds; float eff; bool attr_set; };

#define SH_KCFG(BM, BN, EFF) { BM, BN, { k_gemm<BM, BN, true, false>, k_gemm<BM, BN, true, true> }, \
                               { k_gemm<BM, BN, false, false>, k_gemm<BM, BN, false, true> }, Cfg<BM, BN>::LDS, EFF, false }
KCfg g_cfgs[] = {
    SH_KCFG(256, 256, 0.75f),
    SH_KCFG(256, 128, 0.65f),
    SH_KCFG(128, 256, 0.65f),
    SH_KCFG(128, 192, 0.60f),
    SH_KCFG(128, 128, 0.50f),
    SH_KCFG(64, 64, 0.20f),
};
#undef SH_KCFG
constexpr int kNumCfg = sizeof(g_cfgs) / sizeof(g_cfgs[0]);

int env_int(const char *name, int dflt) {
    const char *e = getenv(name);
    return (e && *e) ? atoi(e) : dflt;
}

// Estimated seconds of config c for an (M, N, K) problem cut into `splits` K ranges: rounds of tiles
// over the CUs at the config's sustained MFMA fraction, plus the split-K partial traffic.
double est_time(const KCfg &c, uint32_t M, uint32_t N, uint32_t K, uint32_t splits, int cus) {
    const double tiles = (double)sh_cdiv(M, c.bm) * sh_cdiv(N, c.bn) * splits;
    const double rounds = std::ceil(tiles / cus);
    const double k_len = (double)sh_cdiv(sh_cdiv(std::max<uint32_t>(K, 1), splits), BK) * BK;
    double t = rounds * c.bm * c.bn * k_len / (c.eff * 2048.0 * 2.4e9);
    if (splits > 1) t += ((double)splits * M * N * 8.0 + (double)M * N * 2.0) / 5e12 + 4e-6;
    return t;
}

struct Plan { int cfg; uint32_t splits; };

Plan choose(uint32_t M, uint32_t N, uint32_t K, bool vec, uint32_t want_splits) {
    const int cus = sh_num_cus() > 0 ? sh_num_cus() : 256;
    Plan best{4, 1};
    double bt = 1e300;
    for (int i = 0; i < kNumCfg; ++i) {
        if (!vec && g_cfgs[i].bm * g_cfgs[i].bn > 128 * 128) continue;
        uint32_t lo = 1, hi = 1;
        if (want_splits) lo = hi = want_splits;
        else hi = std::max<uint32_t>(1, std::min<uint32_t>(8, K / 512));
        for (uint32_t s = lo; s <= hi; ++s) {
            const double tt = est_time(g_cfgs[i], M, N, K, s, cus);
            if (tt < bt * 0.97) { bt = tt; best = {i, s}; }
        }
    }
    const int fc = env_int("SH_GEMM_CFG", -1);
    if (fc >= 0 && fc < kNumCfg && (vec || g_cfgs[fc].bm * g_cfgs[fc].bn <= 128 * 128)) best.cfg = fc;
    const int fs = env_int("SH_GEMM_SPLITS", 0);
    if (fs > 0 && !want_splits) best.splits = (uint32_t)fs;
    return best;
}

struct GemmReq {
    uint64_t x, w, z; uint32_t M, N, K; uint32_t ldx, ldw, ldz;
    uint32_t accumulate; const sh_gemm_epi *epi; uint32_t splits; bool mesh;
};

int launch(const GemmReq &r, const char *name) {
    if (r.M == 0 || r.N == 0) return 0;
    const sh_gemm_epi *e = r.epi;
    const uint64_t bias = e ? e->bias : 0, res = e ? e->residual : 0;
    const uint32_t ldr = e ? e->ldr : 0;
    const bool vec = r.N % 8 == 0 && r.K % 8 == 0 && r.ldx % 8 == 0 && r.ldw % 8 == 0 && r.ldz % 8 == 0 &&
                     sh_aligned16(r.x) && sh_aligned16(r.w) && sh_aligned16(r.z) &&
                     (!res || (ldr % 8 == 0 && sh_aligned16(res))) && (!bias || (bias & 3) == 0);
    Plan p = choose(r.M, r.N, r.K, vec, r.splits);
    if (r.mesh) p.splits = 1;
    KCfg &c = g_cfgs[p.cfg];
    uint32_t splits = std::max<uint32_t>(1, std::min<uint32_t>(p.splits, sh_cdiv(std::max<uint32_t>(r.K, 1), BK)));
    const uint32_t kps = sh_cdiv(sh_cdiv(std::max<uint32_t>(r.K, 1), splits), BK) * BK;
    splits = sh_cdiv(std::max<uint32_t>(r.K, 1), kps);         // no empty trailing split

    GemmArgs a{};
    a.x = (const uint16_t *)r.x; a.w = (const uint16_t *)r.w; a.z = (uint16_t *)r.z;
    a.bias = (const void *)bias; a.res = (const uint16_t *)res;
    a.ldx = r.ldx; a.ldw = r.ldw; a.ldz = r.ldz; a.ldr = ldr;
    a.M = r.M; a.N = r.N; a.K = r.K; a.kps = kps;
    a.tiles_m = sh_cdiv(r.M, c.bm); a.tiles_n = sh_cdiv(r.N, c.bn); a.splits = splits;
    a.accumulate = r.accumulate; a.bias_fp32 = (e && e->bias_fmt == SH_BIAS_FP32) ? 1 : 0; a.act = e ? e->act : 0;
    const uint64_t nblk64 = (uint64_t)a.tiles_m * a.tiles_n * splits;
    if (nblk64 > 0x7FFFFFFFull) { sh_set_error(-1, "[%s] problem too large", name); return -1; }
    const uint32_t nblk = (uint32_t)nblk64;
    const int X = sh_num_xcds();
    a.xcd_groups = (X > 1 && nblk % (uint32_t)X == 0) ? (uint32_t)X : 1;

    hipStream_t st = sh_stream();
    const bool split = splits > 1;
    KernelFn fn = vec ? c.vec[split] : c.scalar[split];
    if (!c.attr_set) {
        for (int v = 0; v < 2; ++v) {
            (void)hipFuncSetAttribute((const void *)c.vec[v], hipFuncAttributeMaxDynamicSharedMemorySize, (int)c.lds);
            (void)hipFuncSetAttribute((const void *)c.scalar[v], hipFuncAttributeMaxDynamicSharedMemorySize, (int)c.lds);
        }
        c.attr_set = true;
    }
    if (split) {
        const size_t ws = (size_t)splits * r.M * r.N * sizeof(float);
        a.part = (float *)sh_workspace(ws);
        if (!a.part) return SH_EHIP;
    }
    hipLaunchKernelGGL(fn, dim3(nblk), dim3(256), c.lds, st, a);
    if (!sh_launch_ok(name)) return SH_EHIP;
    if (split) {
        const bool rvec = vec;
        const uint32_t per_row = rvec ? r.N / 8 : r.N;
        const uint64_t items = (uint64_t)r.M * per_row;
        if (items > 0xFFFFFF00ull) { sh_set_error(-1, "[%s] problem too large", name); return -1; }
        const ShDiv div = sh_make_div(per_row);
        if (rvec) hipLaunchKernelGGL(k_splitk_reduce<true>, dim3(sh_cdiv((uint32_t)items, 256)), dim3(256), 0, st, a, div, per_row, (uint32_t)items);
        else hipLaunchKernelGGL(k_splitk_reduce<false>, dim3(sh_cdiv((uint32_t)items, 256)), dim3(256), 0, st, a, div, per_row, (uint32_t)items);
        if (!sh_launch_ok(name)) return SH_EHIP;
    }
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

int sh_gemm_ex(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
               uint32_t ldx, uint32_t ldw, uint32_t ldz, const sh_gemm_cfg *cfg, const sh_gemm_epi *epi) {
    sh_gemm_cfg c;
    cfg_fill(&c, cfg);
    if (!x || !w || !z) { sh_set_error(-1, "[sh_gemm_ex] NULL tensor address"); return -1; }
    if (c.fmt != SH_FP16) { sh_set_error(-1, "[sh_gemm_ex] fmt %u: only SH_FP16 is implemented", c.fmt); return -1; }
    if (epi && epi->residual && epi->ldr < N) { sh_set_error(-1, "[sh_gemm_ex] ldr %u < N %u", epi->ldr, N); return -1; }
    if (epi && epi->act > SH_ACT_GELU) { sh_set_error(-1, "[sh_gemm_ex] unknown act %u", epi->act); return -1; }
    GemmReq r{x, w, z, M, N, K, ldx, ldw, ldz, c.accumulate, epi, epi ? epi->splits : 1u, false};
    return launch(r, "sh_gemm_ex");
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
