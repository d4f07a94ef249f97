// Fused multi-head attention (reference runtime/sh_attention.inc.c:55-243, semantics of
// tests/gvsoc/run.py:921-934): o_h = softmax(scale * q_h k_h^T) v_h, head h = columns [h*dh, (h+1)*dh).
//
// Flash-style on gfx950: a 256-thread workgroup owns 128 queries of one (sequence, head); each wavefront
// owns 32 of them and walks the keys in blocks of 64 with an online softmax (running max m and sum l per
// query), so the S x S scores never leave the CU and S is unbounded.
//  - Scores are computed transposed, S^T[key, q] = K . Q^T, with v_mfma_f32_32x32x16_f16: A = K rows
//    (64 keys as two 32-row tiles, dh contiguous, staged in LDS), B = Q^T (each lane keeps its query's
//    dh values in registers for the whole kernel). The accumulator then gives every lane 16 keys of one
//    query per tile, so max / sum statistics are lane-local plus one exchange with lane ^ 32.
//  - O^T[d, q] = V^T . P^T: the softmax numerators P (fp16) are the B operand straight from the score
//    accumulators; V is transposed into LDS (8 x 8 register transposes) with its keys stored in the order
//    that matches the accumulator layout (within 16 keys: 0-3, 8-11, 4-7, 12-15), so every MFMA operand is
//    one 16-byte LDS read.
//  - K/V blocks are double-buffered in LDS; the next block is loaded from HBM while the current one is used.
//  - exp is 2^(c s - m) with c = scale * log2(e) on the hardware exp2; O is normalised by 1/l at the end,
//    staged in LDS and written as 16-byte row chunks.
// Heads with dh <= 128 use this kernel (dh padded to 64 or 128 with zeros); wider heads use a simple
// per-query kernel.
#include "sh_common.h"
#include <hip/hip_ext.h>
#include <algorithm>
#include <chrono>
#include <type_traits>

namespace {

constexpr int KB = 64;           // keys per block
constexpr int QPW = 32;          // queries per wavefront
constexpr int QPB = 128;         // queries per workgroup

struct AttnArgs {
    const uint16_t *q, *k, *v;
    uint16_t *o;
    uint64_t ldq, ldk, ldv, ldo;
    uint64_t bsq, bsk, bsv, bso;    // batch strides (elements)
    uint32_t S, dh;
    float c;                        // scale * log2(e)
    const uint16_t *tok;            // token classes of the S positions (sh_ops.h:277-282), or null: no mask
    uint32_t grp;                   // query heads per key/value head (GQA); 1 for plain multi-head attention
    uint32_t xcds;                  // > 1: the query blocks of one head run on one XCD (see attn_item)
    uint64_t mx, mgx, mgy;          // with xcds > 1: ceil(2^32 / d) for d = xcds, gridDim.x, gridDim.y (attn_item)
    // sh_attention_batched_prefetch: two ranges of 64-byte lines (line-aligned bases, line counts) that k_flash3
    // reads into the caches while it runs; zero counts: none
    const uint8_t *pf0, *pf1;
    uint32_t pfl0, pfl1;
};

// Work item of a workgroup: (query block, head, sequence). Dispatch deals workgroups round-robin over the XCDs,
// and every query block of a head reads the same K / V, so with `xcds` > 1 the flat block id L is remapped to
// keep a head's query blocks on one XCD, back to back (L % X picks the XCD, L / X the position in its queue),
// and the second block's K / V reads hit that XCD's L2. Needs (heads x sequences) % X == 0.
// (the quotients by multiply-high with the host's ceil(2^32 / d), exact for n d < 2^32, which the host checks: scalar
// instructions where a division would take ~10 vector ones)
__device__ __forceinline__ uint32_t attn_div(uint32_t n, uint64_t m) { return (uint32_t)(((uint64_t)n * m) >> 32); }
__device__ __forceinline__ void attn_item(const AttnArgs &a, uint32_t &qb, uint32_t &h, uint32_t &b) {
    qb = blockIdx.x; h = blockIdx.y; b = blockIdx.z;
    if (a.xcds > 1) {
        const uint32_t gx = gridDim.x, gy = gridDim.y;
        const uint32_t L = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
        const uint32_t j = attn_div(L, a.mx), jx = attn_div(j, a.mgx);
        const uint32_t hb = jx * a.xcds + (L - j * a.xcds), hy = attn_div(hb, a.mgy);
        qb = j - jx * gx; h = hb - hy * gy; b = hy;
    }
}
constexpr uint32_t kLlmPad = 0xFFFFu;   // SH_LLM_PAD: a padding position

template <int DH>
__device__ __forceinline__ uint32_t kswz(uint32_t r) {
    if (DH == 128) return r & 15u;
    return (r ^ (r >> 3)) & 7u;
}
__device__ __forceinline__ uint32_t vswz(uint32_t r) { return (r ^ (r >> 3)) & 7u; }
__device__ __forceinline__ uint32_t comp4(const uint4 &q, int i) { return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w; }

// 8 halves of row r starting at column c of a [*, ld] matrix; zero outside rows < rmax, cols < cmax.
template <bool VEC>
__device__ __forceinline__ uint4 ld8(const uint16_t *p, uint64_t ld, uint32_t r, uint32_t c, uint32_t rmax, uint32_t cmax) {
    if (VEC) {
        if (r < rmax && c < cmax) return *(const uint4 *)(p + (uint64_t)r * ld + c);
        return make_uint4(0, 0, 0, 0);
    }
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (r < rmax && c + e < cmax) ? p[(uint64_t)r * ld + c + e] : 0u;
    return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
}

template <int DH, bool VEC>
__global__ __launch_bounds__(256) void k_flash(AttnArgs a) {
    constexpr int DC = DH / 8;                 // 16-byte chunks per K row
    constexpr int NS = DH / 16;                // QK k-substeps
    constexpr int DT = DH / 32;                // O^T row tiles
    constexpr int K_PER_T = KB * DC / 256;     // K chunks per thread per block
    constexpr int K_ELEMS = KB * DC;           // uint4 per K stage
    constexpr int V_ELEMS = DH * 8;            // uint4 per V^T stage (DH rows x 8 chunks)
    __shared__ uint4 smem[2 * (K_ELEMS + V_ELEMS)];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = lane >> 5, r32 = lane & 31;
    const uint32_t b = blockIdx.z, h = blockIdx.y;
    const uint32_t S = a.S, dh = a.dh;
    const uint16_t *Q = a.q + b * a.bsq + (uint64_t)h * dh;
    const uint16_t *Kp = a.k + b * a.bsk + (uint64_t)(h / a.grp) * dh;
    const uint16_t *Vp = a.v + b * a.bsv + (uint64_t)(h / a.grp) * dh;
    uint16_t *O = a.o + b * a.bso + (uint64_t)h * dh;
    const uint32_t qw0 = blockIdx.x * QPB + wave * QPW;    // first query of this wavefront
    const uint32_t myq = qw0 + r32;

    // Q^T operand: substep s, lane group g -> dh [16 s + 8 g, +8)
    sh_h8 qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = __builtin_bit_cast(sh_h8, ld8<VEC>(Q, a.ldq, myq, 16 * s + 8 * g, S, dh));

    sh_f16v oacc[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) oacc[i] = sh_f16v{};
    float m_run = -INFINITY, l_run = 0.f;

    uint4 rk[K_PER_T], rv[8];
    const bool vload = t < DH;                 // V: one (8 keys x 8 dh) block per thread
    const int vkc = t & 7, vdc = t >> 3;
    const uint32_t nkb = (S + KB - 1) / KB;

    auto gload = [&](uint32_t kb) {
        const uint32_t k0 = kb * KB;
#pragma unroll
        for (int i = 0; i < K_PER_T; ++i) {
            const int c = t + 256 * i, key = c / DC, kc = c % DC;
            rk[i] = ld8<VEC>(Kp, a.ldk, k0 + key, 8 * kc, S, dh);
        }
        if (vload) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {      // key-chunk vkc = 2 * b16 + gg holds keys 16 b16 + 4 gg + {0..3, 8..11}
                const int key = 16 * (vkc >> 1) + 4 * (vkc & 1) + (i & 3) + 8 * (i >> 2);
                rv[i] = ld8<VEC>(Vp, a.ldv, k0 + key, 8 * vdc, S, dh);
            }
        }
    };
    auto sstore = [&](int st) {
        uint4 *sk = smem + st * (K_ELEMS + V_ELEMS);
        uint4 *sv = sk + K_ELEMS;
#pragma unroll
        for (int i = 0; i < K_PER_T; ++i) {
            const int c = t + 256 * i, key = c / DC, kc = c % DC;
            sk[key * DC + (kc ^ kswz<DH>(key))] = rk[i];
        }
        if (vload) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {      // V^T row d = 8 vdc + j: column j of the 8 loaded rows
                uint32_t o4[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const uint32_t lo = comp4(rv[2 * p], j >> 1), hi = comp4(rv[2 * p + 1], j >> 1);
                    o4[p] = (j & 1) ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
                }
                const int d = 8 * vdc + j;
                sv[d * 8 + (vkc ^ vswz(d))] = make_uint4(o4[0], o4[1], o4[2], o4[3]);
            }
        }
    };

    if (nkb > 0) {
        gload(0);
        sstore(0);
    }
    __syncthreads();
    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const int st = kb & 1;
        if (kb + 1 < nkb) gload(kb + 1);
        const uint4 *sk = smem + st * (K_ELEMS + V_ELEMS);
        const uint4 *sv = sk + K_ELEMS;

        // S^T tiles: keys [32 tt, 32 tt + 32) of this block x this wavefront's 32 queries
        sh_f16v sacc[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            sacc[tt] = sh_f16v{};
            const uint32_t key = 32 * tt + r32;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const sh_h8 kf = __builtin_bit_cast(sh_h8, sk[key * DC + ((2 * s + g) ^ kswz<DH>(key))]);
                sacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], sacc[tt], 0, 0, 0);
            }
        }
        // lane (q, g) holds key 64 kb + 32 tt + 8 (r / 4) + 4 g + r % 4 in sacc[tt][r]
        const bool masked = (kb + 1) * KB > S;   // last block of a ragged S: keys >= S take no weight
        if (masked) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (kb * KB + 32 * tt + 8 * (r >> 2) + 4 * g + (r & 3) >= S) sacc[tt][r] = a.c >= 0.f ? -INFINITY : INFINITY;
        }
        float mb;
        if (a.c >= 0.f) {
            mb = -INFINITY;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) mb = fmaxf(mb, sacc[tt][r]);
            mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
        } else {
            mb = INFINITY;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) mb = fminf(mb, sacc[tt][r]);
            mb = fminf(mb, __shfl_xor(mb, 32, 64));
        }
        const float m_new = fmaxf(m_run, a.c * mb);
        const float alpha = sh_fast_exp2(m_run - m_new);
        m_run = m_new;
        float psum = 0.f;
        sh_h8 pf[4];                           // P^T operand of PV substep s' (keys [16 s', 16 s' + 16))
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float p = sh_fast_exp2(fmaf(sacc[tt][r], a.c, -m_new));
                if (masked && kb * KB + 32 * tt + 8 * (r >> 2) + 4 * g + (r & 3) >= S) p = 0.f;
                psum += p;
                pf[2 * tt + (r >> 3)][r & 7] = (_Float16)p;
            }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const uint32_t d = 32 * dt + r32;
#pragma unroll
            for (int sp = 0; sp < 4; ++sp) {
                const sh_h8 vf = __builtin_bit_cast(sh_h8, sv[d * 8 + ((2 * sp + g) ^ vswz(d))]);
                oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[sp], oacc[dt], 0, 0, 0);
            }
        }
        if (kb + 1 < nkb) sstore((kb + 1) & 1);
        __syncthreads();
    }

    // normalise and write: lane (q, g) holds O[q][32 dt + 8 (r / 4) + 4 g + r % 4] in oacc[dt][r]
    const float l = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = 1.f / l;
    uint16_t *so = (uint16_t *)smem + wave * (QPW * DH);     // [32 q][DH] per wavefront, chunk c at c ^ (q & 7)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int d0 = 32 * dt + 8 * rb + 4 * g;
            const uint32_t lo = (uint32_t)sh_dev_f2h(oacc[dt][4 * rb] * inv) | ((uint32_t)sh_dev_f2h(oacc[dt][4 * rb + 1] * inv) << 16);
            const uint32_t hi = (uint32_t)sh_dev_f2h(oacc[dt][4 * rb + 2] * inv) | ((uint32_t)sh_dev_f2h(oacc[dt][4 * rb + 3] * inv) << 16);
            const int ch = (d0 >> 3) ^ (r32 & 7);
            *(uint2 *)(so + r32 * DH + ch * 8 + (d0 & 7)) = make_uint2(lo, hi);
        }
    __syncthreads();
    for (int c = lane; c < QPW * DC; c += 64) {
        const int row = c / DC, ch = c % DC;
        const uint32_t qq = qw0 + row, col = 8 * ch;
        if (qq >= S || col >= dh) continue;
        const uint4 val = ((const uint4 *)so)[row * DC + (ch ^ (row & 7))];
        if (VEC) {
            *(uint4 *)(O + (uint64_t)qq * a.ldo + col) = val;
        } else {
            for (int e = 0; e < 8 && col + e < dh; ++e) O[(uint64_t)qq * a.ldo + col + e] = (uint16_t)(comp4(val, e >> 1) >> (16 * (e & 1)));
        }
    }
}

// ---- V layout of the DMA kernels (dh == 64 or 128, 16-byte aligned operands) -------------------------------
// K and V key blocks are copied HBM -> LDS by global_load_lds_dwordx4. V stays in its natural [key][d] layout and
// the O^T MFMA reads its A operand (8 keys of one d per lane) with two ds_read_b64_tr_b16: lane group g of a 16-key
// substep supplies keys 4g..4g+3 and 8+4g..8+4g+3, the order in which the score accumulators hold P.
// V rows are DC chunks wide; chunk c of row k sits at c ^ vfw(k) so a transpose read's 4 rows x 64 bytes
// land on distinct banks (row pitch 128 B: alternate rows share a bank half; 256 B: every row starts at bank 0)
template <int DH>
__device__ __forceinline__ uint32_t vfw(uint32_t k) { return DH == 128 ? 4u * (k & 3u) : 4u * ((k >> 1) & 1u); }

// Profiling stamp: the 100 MHz real-time counter into slot i of the stamp buffer (a vector store).
__device__ __forceinline__ void attn_stamp(uint64_t *stamp, bool on, int i) {
    if (on) {
        const uint64_t t = __builtin_amdgcn_s_memrealtime();
        __builtin_nontemporal_store(t, stamp + i);
    }
}

// Two-pass flash attention for dh 64 / 128 (aligned heads with a token mask or a scale that does not
// fold, |c| > 1; SH_ATTN_IMPL=2 selects it for every aligned head). On CDNA the softmax
// VALU work, not the MFMA work, bounds attention, so the row maximum is found first in a cheap pass over the
// keys (S^T = K . Q^T on MFMA, then max3 only); the second pass recomputes the scores and, with the final
// maximum known, needs no running rescale of O or l: p = 2^(c s - m), P (fp16) feeds O^T += V^T . P^T, and
// the row sums l are the sums of the fp16 numerators the PV product used (v_dot2_f32_f16 with ones, fp32).
// Masking of keys past S happens only in the last, partial key block. LDS fragment reads are issued ahead of
// the MFMAs that use them (two ahead for K, one for V), so a read's latency overlaps earlier MFMAs.
// FOLD (|c| <= 1, so c q stays in fp16 range): the softmax VALU work shrinks by folding c and m into the score
// MFMAs. The query fragments are scaled once, q' = r16(c q), so the scores come out as c s (pass 1 then takes
// a plain maximum for either sign of c), and pass 2 adds one more 16-k MFMA step per score tile whose
// operands are ones (keys) and -m_hi, -m_lo (queries; m_hi = r16(m), m_lo = r16(m - m_hi)), so the
// accumulator already holds c s - m and p = 2^acc needs no VALU multiply-add. An error in m common to a
// query's row scales its numerators and its row sum alike and cancels in O / l; the rounding of c q changes
// each exponent by ~1e-4 relative.
// Occupancy: with a 2-stage ring (32 KB of LDS) a dh = 64 workgroup fits in 168 registers per lane, so three
// workgroups share a CU (12 waves); the encoder's 768 (sequence, head, query block) workgroups then run in one round.
template <int DH, int NST, bool MASK, bool FOLD>
__global__ __launch_bounds__(256, DH == 64 ? 3 : 2) void k_flash2(AttnArgs a, uint64_t *stamp) {
    constexpr int DC = DH / 8, NS = DH / 16, DT = DH / 32;
    constexpr int KCH = KB * DC;                     // 16-byte chunks per K (or V) block
    constexpr int KR = KCH / 256;                    // DMA rounds per thread per block, per operand
    constexpr uint32_t STAGE = 2u * KCH * 16u;       // K block then V block
    static_assert(KCH % 256 == 0 && NST >= 2, "attention tiling");
    __shared__ uint4 smem[NST * 2 * KCH];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = lane >> 5, r32 = lane & 31;
    const int q4 = lane >> 4, iq = lane & 15;
    uint32_t qb, h, b;
    attn_item(a, qb, h, b);
    const uint32_t S = a.S;
    const uint16_t *Q = a.q + b * a.bsq + (uint64_t)h * DH;
    const uint16_t *Kp = a.k + b * a.bsk + (uint64_t)(h / a.grp) * DH;
    const uint16_t *Vp = a.v + b * a.bsv + (uint64_t)(h / a.grp) * DH;
    uint16_t *O = a.o + b * a.bso + (uint64_t)h * DH;
    const uint32_t qw0 = qb * QPB + wave * QPW, myq = qw0 + r32;
    const uint32_t nkb = (S + KB - 1) / KB;
    const bool ragged = S % KB != 0;                 // the last key block is partial
    // stamps (profile): 0-2 start, 3-4 pass 1 done (maximum known), 5 pass 2 done, 6 stored; 7 first workgroup
    const bool last = stamp && t == 0 && qb == gridDim.x - 1 && h == gridDim.y - 1 && b == gridDim.z - 1;
    attn_stamp(stamp, stamp && t == 0 && qb == 0 && h == 0 && b == 0, 7);
    attn_stamp(stamp, last, 0);
    attn_stamp(stamp, last, 1);
    attn_stamp(stamp, last, 2);
    // token mask (MASK): key j is allowed for this lane's query iff tok[j] <= tok[query]; a padding query (or
    // one with no allowed key, found in pass 1) averages V uniformly over the S keys
    const uint32_t tq = MASK ? (myq < S ? (uint32_t)a.tok[myq] : kLlmPad) : 0u;
    bool uni = MASK && tq == kLlmPad;

    const uint16_t *kcol[KR];
    const uint16_t *vcol[KR];
    uint32_t kkey[KR];
#pragma unroll
    for (int r = 0; r < KR; ++r) {
        const uint32_t p = r * 256 + wave * 64 + lane, key = p / DC, pc = p % DC;
        kkey[r] = key;
        kcol[r] = Kp + 8 * (pc ^ kswz<DH>(key));
        vcol[r] = Vp + 8 * (pc ^ vfw<DH>(key));
    }
    const uint32_t lds0 = sh_lds_addr(smem);
    const uint32_t wave_off = (uint32_t)__builtin_amdgcn_readfirstlane(wave * 64 * 16);
    auto issue = [&](uint32_t kb, int stage, bool with_v) {
        const uint32_t st = lds0 + (uint32_t)stage * STAGE;
        const uint32_t k0 = kb * KB;
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            const uint64_t row = min(k0 + kkey[r], S - 1);                      // rows past S read row S-1
            sh_lds_dma16(kcol[r] + row * a.ldk, st + r * 4096 + wave_off);
            if (with_v) sh_lds_dma16(vcol[r] + row * a.ldv, st + KCH * 16 + r * 4096 + wave_off);
        }
    };

    sh_h8 qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = __builtin_bit_cast(sh_h8, ld8<true>(Q, a.ldq, myq, 16 * s + 8 * g, S, DH));
    if constexpr (FOLD) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[s][e] = (_Float16)((float)qf[s][e] * a.c);
    }
    // FOLD: operands of the bias step (k elements 0 and 1 of lane group 0): ones for every key, -m_hi, -m_lo
    // of this lane's query (set once m is known)
    sh_h8 kbias = {}, qbias = {};
    if (FOLD && g == 0) { kbias[0] = (_Float16)1.0f; kbias[1] = (_Float16)1.0f; }

    // S^T tile pair of key block in stage st: sacc[tt][r] = s(key 32 tt + 8 (r/4) + 4 g + r%4, query r32)
    // (FOLD: c s, and with bias, c s - m). The 2 NS K fragments are read two MFMAs ahead of their use (the two
    // tiles' chains interleaved), so each LDS read has two MFMAs to land in.
    auto kfrag = [&](const uint4 *sk, int i) -> sh_h8 {        // fragment i: substep i / 2 of tile i % 2
        const uint32_t key = 32 * (i & 1) + r32;
        return __builtin_bit_cast(sh_h8, sk[key * DC + ((2 * (i >> 1) + g) ^ kswz<DH>(key))]);
    };
    auto scores = [&](int st, sh_f16v (&sacc)[2], bool bias) {
        const uint4 *sk = smem + st * 2 * KCH;
        constexpr int NI = 2 * NS;
        sh_h8 kf[3];
        kf[0] = kfrag(sk, 0);
        kf[1] = kfrag(sk, 1);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            sacc[tt] = sh_f16v{};
            if (FOLD && bias) sacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kbias, qbias, sacc[tt], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if (i + 2 < NI) kf[(i + 2) % 3] = kfrag(sk, i + 2);
            sacc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[i % 3], qf[i >> 1], sacc[i & 1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto key_of = [&](uint32_t kb, int tt, int r) { return kb * KB + 32 * tt + 8 * (r >> 2) + 4 * g + (r & 3); };
    auto key_ok = [&](uint32_t kb, int tt, int r) {
        const uint32_t key = key_of(kb, tt, r);
        if (!MASK) return key < S;
        return key < S && (uint32_t)a.tok[min(key, S - 1)] <= tq;
    };

    // ---- pass 1: extreme of s over all keys (max for c >= 0, min for c < 0; FOLD: max of c s), K blocks only ----
    const bool pos = FOLD || a.c >= 0.f;
#pragma unroll
    for (int s = 0; s < NST - 1; ++s) issue(min((uint32_t)s, nkb - 1), s, false);
    float ext = pos ? -INFINITY : INFINITY;
    for (uint32_t kb = 0; kb < nkb; ++kb) {
        sh_wait_vmcnt<(NST - 2) * KR>();
        __syncthreads();
        issue(min(kb + NST - 1, nkb - 1), (int)((kb + NST - 1) % NST), false);
        sh_f16v sacc[2];
        scores((int)(kb % NST), sacc, false);
        if (MASK || (ragged && kb == nkb - 1)) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (!key_ok(kb, tt, r)) sacc[tt][r] = pos ? -INFINITY : INFINITY;
        }
        if (pos) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) ext = fmaxf(ext, sacc[tt][r]);
        } else {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) ext = fminf(ext, sacc[tt][r]);
        }
    }
    ext = pos ? fmaxf(ext, __shfl_xor(ext, 32, 64)) : fminf(ext, __shfl_xor(ext, 32, 64));
    if (MASK) uni = uni || ext == -INFINITY;
    const float m = (MASK && uni) ? 0.f : (FOLD ? ext : a.c * ext);   // max over keys of c s
    if (FOLD && g == 0) {
        const _Float16 mh = (_Float16)m;
        qbias[0] = -mh;
        qbias[1] = -(_Float16)(m - (float)mh);
    }
    sh_wait_vmcnt<0>();                            // the ring is idle before pass 2 refills it
    __syncthreads();
    attn_stamp(stamp, last, 3);
    attn_stamp(stamp, last, 4);

    // ---- pass 2: p = 2^(c s - m); O^T += V^T P^T; l += 1^T P^T ----
    sh_f16v oacc[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) oacc[i] = sh_f16v{};
    float lsum = 0.f;                                // this lane's keys' fp16 numerators, summed in fp32
    const sh_h2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int s = 0; s < NST - 1; ++s) issue(min((uint32_t)s, nkb - 1), s, true);
    for (uint32_t kb = 0; kb < nkb; ++kb) {
        sh_wait_vmcnt<(NST - 2) * 2 * KR>();
        __syncthreads();
        issue(min(kb + NST - 1, nkb - 1), (int)((kb + NST - 1) % NST), true);
        const int st = (int)(kb % NST);
        sh_f16v sacc[2];
        scores(st, sacc, true);
        sh_h8 pf[4];
        const bool tail = ragged && kb == nkb - 1;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float p = FOLD ? sh_fast_exp2(sacc[tt][r]) : sh_fast_exp2(fmaf(sacc[tt][r], a.c, -m));
                if (MASK) {
                    if (uni) p = key_of(kb, tt, r) < S ? 1.f : 0.f;
                    else if (!key_ok(kb, tt, r)) p = 0.f;
                } else if (tail && !key_ok(kb, tt, r)) {
                    p = 0.f;
                }
                pf[2 * tt + (r >> 3)][r & 7] = (_Float16)p;
            }
        const uint32_t vbase = lds0 + (uint32_t)st * STAGE + KCH * 16;
        // V^T fragment j: substep j / DT, d tile j % DT (consecutive MFMAs alternate accumulators); read one ahead
        auto vfrag = [&](int j) -> sh_h8 {
            const int sp = j / DT, dt = j % DT;
            const uint32_t d = 32 * dt + 16 * (q4 & 1) + 4 * (iq & 3);
            const uint32_t k0 = 16 * sp + 4 * g + (iq >> 2), k1 = k0 + 8;
            const sh_s4 lo = sh_ds_read_tr(vbase + k0 * (DH * 2) + 16 * ((d >> 3) ^ vfw<DH>(k0)) + 2 * (d & 7));
            const sh_s4 hi = sh_ds_read_tr(vbase + k1 * (DH * 2) + 16 * ((d >> 3) ^ vfw<DH>(k1)) + 2 * (d & 7));
            return __builtin_bit_cast(sh_h8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        };
        constexpr int NJ = 4 * DT;
        sh_h8 vq[2];
        vq[0] = vfrag(0);
#pragma unroll
        for (int sp = 0; sp < 4; ++sp) {
            const uint4 w = __builtin_bit_cast(uint4, pf[sp]);
            lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(sh_h2, w.x), one2, lsum, false);
            lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(sh_h2, w.y), one2, lsum, false);
            lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(sh_h2, w.z), one2, lsum, false);
            lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(sh_h2, w.w), one2, lsum, false);
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            if (j + 1 < NJ) vq[(j + 1) & 1] = vfrag(j + 1);
            oacc[j % DT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vq[j & 1], pf[j / DT], oacc[j % DT], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    sh_wait_vmcnt<0>();      // clamped tail loads land before the LDS is reused below
    __syncthreads();
    attn_stamp(stamp, last, 5);

    const float inv = 1.f / (lsum + __shfl_xor(lsum, 32, 64));   // lanes g = 0, 1 hold complementary keys
    uint16_t *so = (uint16_t *)(smem + 2 * KCH) + wave * (QPW * DH);     // this wave's query rows, now free
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int d0 = 32 * dt + 8 * rb + 4 * g;
            const uint32_t lo = (uint32_t)sh_dev_f2h(oacc[dt][4 * rb] * inv) | ((uint32_t)sh_dev_f2h(oacc[dt][4 * rb + 1] * inv) << 16);
            const uint32_t hi = (uint32_t)sh_dev_f2h(oacc[dt][4 * rb + 2] * inv) | ((uint32_t)sh_dev_f2h(oacc[dt][4 * rb + 3] * inv) << 16);
            const int ch = (d0 >> 3) ^ (r32 & 7);
            *(uint2 *)(so + r32 * DH + ch * 8 + (d0 & 7)) = make_uint2(lo, hi);
        }
    __builtin_amdgcn_s_waitcnt(0xC07F);              // lgkmcnt(0): the wave's own staging is complete
    __builtin_amdgcn_wave_barrier();
    for (int c = lane; c < QPW * DC; c += 64) {
        const int row = c / DC, ch = c % DC;
        const uint32_t qq = qw0 + row;
        if (qq >= S) continue;
        *(uint4 *)(O + (uint64_t)qq * a.ldo + 8 * ch) = ((const uint4 *)so)[row * DC + (ch ^ (row & 7))];
    }
    attn_stamp(stamp, last, 6);
}

// One-pass variant of k_flash2 (the default for aligned dh 64 / 128 heads whose scale folds, |c| <= 1, without a
// token mask): each key block's scores come out of the MFMAs already shifted by the query's reference m (the FOLD
// bias step: ones x (-m_hi, -m_lo)), so p = 2^acc. m starts at 0 and moves to the first block's maximum when that
// lies more than kTau (log2 units) from 0; a later block is first tested by its numerators' sum per lane (32 keys,
// formed for the row sum anyway), and only when that exceeds 32 x 2^kTau is its maximum formed and m moved for the
// queries whose maximum exceeds m by more than kTau. Only then are O and l rescaled by 2^-shift and the block's scores
// computed again with the new bias (a wave-uniform branch, rare for attention inputs of moderate scale). Numerators
// are thus at most 32 x 2^kTau and the largest is at least 2^-kTau, well inside fp16's normal range, and the row sums are the sums of the
// same fp16 numerators the P.V product uses, so O / l is the softmax with every p rounded once. Against k_flash2
// this drops the maximum pass (its score MFMAs, K fragment reads and K DMAs) and the refill of the ring between the
// passes. Same LDS ring, fragment prefetch and occupancy as k_flash2.
constexpr float kTau = 8.f;
template <int DH, int NST, bool PF = false, bool ST = true, bool RAG = true>
__global__ __launch_bounds__(256, DH == 64 ? 3 : 2) void k_flash3(AttnArgs a, uint64_t *stamp) {
    constexpr int DC = DH / 8, NS = DH / 16, DT = DH / 32;
    constexpr int KCH = KB * DC;                     // 16-byte chunks per K (or V) block
    constexpr int KR = KCH / 256;                    // DMA rounds per thread per block, per operand
    constexpr uint32_t STAGE = 2u * KCH * 16u;       // K block then V block
    static_assert(KCH % 256 == 0 && NST == 2, "attention tiling (the key-block loop is unrolled by the two stages)");
    __shared__ uint4 smem[NST * 2 * KCH];
    __shared__ uint4 pf_sink[PF ? 64 : 1];           // destination of the prefetch DMAs (never read)

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = lane >> 5, r32 = lane & 31;
    const int q4 = lane >> 4, iq = lane & 15;
    uint32_t qb, h, b;
    attn_item(a, qb, h, b);
    const uint32_t S = a.S;
    const uint16_t *Q = a.q + b * a.bsq + (uint64_t)h * DH;
    const uint16_t *Kp = a.k + b * a.bsk + (uint64_t)(h / a.grp) * DH;
    const uint16_t *Vp = a.v + b * a.bsv + (uint64_t)(h / a.grp) * DH;
    uint16_t *O = a.o + b * a.bso + (uint64_t)h * DH;
    const uint32_t qw0 = qb * QPB + wave * QPW, myq = qw0 + r32;
    const uint32_t nkb = (S + KB - 1) / KB;
    const bool ragged = RAG && S % KB != 0;       // the last key block is partial (RAG = false: S % 64 == 0, no tail code)
    // stamps (profile): 0-2 start, 3-4 first key block done (the reference m set), 5 all blocks done, 6 stored;
    // 7 first workgroup
    // (ST = false: a launch without a stamp buffer; the stamp code is compiled out)
    const bool last = ST && stamp && t == 0 && qb == gridDim.x - 1 && h == gridDim.y - 1 && b == gridDim.z - 1;
    attn_stamp(stamp, ST && stamp && t == 0 && qb == 0 && h == 0 && b == 0, 7);
    attn_stamp(stamp, last, 0);
    attn_stamp(stamp, last, 1);
    attn_stamp(stamp, last, 2);

    // DMA sources: the block's first row (wave-uniform, scalar registers) plus each lane's 32-bit byte offset of its
    // row and swizzled chunk (the host launches this kernel only when 64 rows of either stride span < 2 GiB)
    uint32_t koff[KR], voff[KR];
#pragma unroll
    for (int r = 0; r < KR; ++r) {
        const uint32_t p = r * 256 + wave * 64 + lane, key = p / DC, pc = p % DC;
        koff[r] = key * (uint32_t)a.ldk * 2 + 16 * (pc ^ kswz<DH>(key));
        voff[r] = key * (uint32_t)a.ldv * 2 + 16 * (pc ^ vfw<DH>(key));
    }
    const uint32_t lds0 = sh_lds_addr(smem);
    const uint32_t wave_off = (uint32_t)__builtin_amdgcn_readfirstlane(wave * 64 * 16);
    auto issue = [&](uint32_t kb, int stage) {
        const uint32_t st = lds0 + (uint32_t)stage * STAGE;
        const uint32_t k0 = kb * KB;
        const char *kbase = (const char *)(Kp + (uint64_t)k0 * a.ldk), *vbase = (const char *)(Vp + (uint64_t)k0 * a.ldv);
        if (k0 + KB <= S) {
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                sh_lds_dma16_s(kbase, koff[r], st + r * 4096 + wave_off);
                sh_lds_dma16_s(vbase, voff[r], st + KCH * 16 + r * 4096 + wave_off);
            }
        } else {                                     // the ragged last block: rows past S read row S - 1
            const uint32_t lim = S - 1 - k0;
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                const uint32_t key = (uint32_t)(r * 256 + wave * 64 + lane) / DC, over = key > lim ? key - lim : 0u;
                sh_lds_dma16_s(kbase, koff[r] - over * (uint32_t)a.ldk * 2, st + r * 4096 + wave_off);
                sh_lds_dma16_s(vbase, voff[r] - over * (uint32_t)a.ldv * 2, st + KCH * 16 + r * 4096 + wave_off);
            }
        }
    };
    // The caller's prefetch ranges (sh_attention_batched_prefetch): one 16-byte DMA per 64-byte line into the sink,
    // a quarter of the lines with each of the first four key blocks, right after that block's next-block DMA, so
    // the reads overlap the blocks' compute and the next block's wait (vmcnt 0) retires them; nothing is read back.
    // (PF: a separate build, so the kernel without ranges keeps its registers)
    const uint32_t pfl = PF ? a.pfl0 + a.pfl1 : 0u, pq = min(nkb, 4u), pfq = (pfl + pq - 1) / pq;
    const uint64_t gthreads = (uint64_t)gridDim.x * gridDim.y * gridDim.z * 256u;
    const uint64_t gid = (((uint64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * 256u + t;
    const uint32_t sink = sh_lds_addr(pf_sink);
    auto prefetch_part = [&](uint32_t kb) {
        if (!PF || pfl == 0 || kb >= pq) return;
        const uint64_t end = min(pfl, (kb + 1) * pfq);
        for (uint64_t j = (uint64_t)kb * pfq + gid; j < end; j += gthreads) {
            const uint8_t *p = j < a.pfl0 ? a.pf0 + j * 64 : a.pf1 + (j - a.pfl0) * 64;
            sh_lds_dma16(p, sink);
        }
    };
#pragma unroll
    for (int s = 0; s < NST - 1; ++s) issue(min((uint32_t)s, nkb - 1), s);

    // query fragments, scaled once by c: the scores come out as c s
    sh_h8 qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = __builtin_bit_cast(sh_h8, ld8<true>(Q, a.ldq, myq, 16 * s + 8 * g, S, DH));
    // (c q as a multiply-add with +0, which reads the fp16 value directly and equals the product but for the sign
    // of a zero, which no score or exponential sees; the empty asm keeps each fp32 value rounded to fp32 before
    // one paired fp16 conversion, so the multiply-add is not fused into a single-rounding conversion)
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float lo = __builtin_fmaf((float)qf[s][e], a.c, 0.f), hi = __builtin_fmaf((float)qf[s][e + 1], a.c, 0.f);
            asm volatile("" : "+v"(lo), "+v"(hi));
            qf[s][e] = (_Float16)lo;
            qf[s][e + 1] = (_Float16)hi;
        }
    // operands of the bias step (k elements 0 and 1 of lane group 0): ones for every key, -m_hi, -m_lo of this
    // lane's query (set from the running maximum)
    sh_h8 kbias = {}, qbias = {};
    if (g == 0) { kbias[0] = (_Float16)1.0f; kbias[1] = (_Float16)1.0f; }
    auto set_bias = [&](float m) {
        if (g == 0) {
            const _Float16 mh = (_Float16)m;
            qbias[0] = -mh;
            qbias[1] = -(_Float16)(m - (float)mh);
        }
    };

    // S^T tile pair of key block in stage st (as k_flash2): sacc[tt][r] = c s(key 32 tt + 8 (r/4) + 4 g + r%4,
    // query r32) [- m with the bias step]; K fragments read two MFMAs ahead
    auto kfrag = [&](const uint4 *sk, int i) -> sh_h8 {
        const uint32_t key = 32 * (i & 1) + r32;
        return __builtin_bit_cast(sh_h8, sk[key * DC + ((2 * (i >> 1) + g) ^ kswz<DH>(key))]);
    };
    // (stage and bias step are compile-time: fragment addresses fold the stage into the read's immediate offset,
    // and without the bias step the first MFMA of each tile starts from a zero accumulator operand)
    auto scores = [&](auto stc, sh_f16v (&sacc)[2], auto bias_c) {
        constexpr bool bias = decltype(bias_c)::value;
        const uint4 *sk = smem + decltype(stc)::value * 2 * KCH;
        constexpr int NI = 2 * NS;
        sh_h8 kf[3];
        kf[0] = kfrag(sk, 0);
        kf[1] = kfrag(sk, 1);
        if constexpr (bias) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) sacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kbias, qbias, sh_f16v{}, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if (i + 2 < NI) kf[(i + 2) % 3] = kfrag(sk, i + 2);
            if (!bias && i < 2) sacc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[i % 3], qf[i >> 1], sh_f16v{}, 0, 0, 0);
            else sacc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[i % 3], qf[i >> 1], sacc[i & 1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    sh_f16v oacc[DT];                                // (set by the first block's P.V MFMAs, which start from zero)
    float lsum = 0.f;                                // this lane's keys' fp16 numerators, summed in fp32
    float mrun = 0.f;                                // reference m of this lane's query (c s units)
    bool biased = false;                             // some lane's m left 0 (wave-uniform): the bias step is needed
    const sh_h2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
    // LDS byte address in stage 0 of each lane's V^T fragment j (rows k0 of its lower half; the upper half's rows
    // k0 + 8 have the same swizzle, vfw reading only the two low bits of k): the loop adds the stage as an immediate
    constexpr int NJ = 4 * DT;
    uint32_t vaddr[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int sp = j / DT, dt = j % DT;
        const uint32_t d = 32 * dt + 16 * (q4 & 1) + 4 * (iq & 3);
        const uint32_t k0 = 16 * sp + 4 * g + (iq >> 2);
        vaddr[j] = lds0 + KCH * 16 + k0 * (DH * 2) + 16 * ((d >> 3) ^ vfw<DH>(k0)) + 2 * (d & 7);
    }
    using Stage0 = std::integral_constant<int, 0>;
    using Stage1 = std::integral_constant<int, 1>;
    using Biased = std::true_type;
    // key block kb, held in ring stage kb % 2 (= the compile-time stage of stc); first_c: kb == 0, a separate build
    // of the step (O and l hold nothing yet: no rescale, and its P.V MFMAs start from a zero accumulator operand)
    auto step = [&](uint32_t kb, auto stc, auto first_c) {
        constexpr int st = decltype(stc)::value;
        constexpr bool first = decltype(first_c)::value;
        sh_wait_vmcnt<(NST - 2) * 2 * KR>();
        __syncthreads();
        issue(min(kb + NST - 1, nkb - 1), (st + NST - 1) % NST);
        prefetch_part(kb);
        sh_f16v sacc[2];
        auto mask_tail = [&]() {
            if (ragged && kb == nkb - 1) {
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (kb * KB + 32 * tt + 8 * (r >> 2) + 4 * g + (r & 3) >= S) sacc[tt][r] = -INFINITY;
            }
        };
        if (biased) scores(stc, sacc, Biased{});
        else scores(stc, sacc, std::false_type{});   // (while every m is 0 the bias step would add zeros)
        mask_tail();
        // V^T fragment j: substep j / DT, d tile j % DT (consecutive MFMAs alternate accumulators)
        auto vfrag = [&](int j) -> sh_h8 {
            const uint32_t at = vaddr[j] + (uint32_t)st * STAGE;
            const sh_s4 lo = sh_ds_read_tr(at);
            const sh_s4 hi = sh_ds_read_tr(at + 8 * (DH * 2));
            return __builtin_bit_cast(sh_h8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        };
        sh_h8 pf[4];                                 // numerators p = 2^acc, fp16, as the P.V MFMA operands
        auto expo = [&]() {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) pf[2 * tt + (r >> 3)][r & 7] = (_Float16)sh_fast_exp2(sacc[tt][r]);
        };
        // The first V fragments are read now and the numerators formed before the maximum test (formed again in
        // the rare case that m moves): the exponentials then hide those reads' latency and the maximum's chain,
        // and each P.V MFMA finds its fragment, read two MFMAs earlier, in registers.
        constexpr int VA = 2;
        sh_h8 vr[VA + 1];
#pragma unroll
        for (int j = 0; j < VA; ++j) vr[j] = vfrag(j);
        expo();
        // this lane's sum of the block's fp16 numerators (fp32 sums, four chains): the row sum's share and, for a
        // later block, the test whether m must move
        auto psum = [&]() -> float {
            float c[4];
#pragma unroll
            for (int sp = 0; sp < 4; ++sp) {
                const uint4 w = __builtin_bit_cast(uint4, pf[sp]);
                c[sp] = __builtin_amdgcn_fdot2(__builtin_bit_cast(sh_h2, w.x), one2, 0.f, false);
                c[sp] = __builtin_amdgcn_fdot2(__builtin_bit_cast(sh_h2, w.y), one2, c[sp], false);
                c[sp] = __builtin_amdgcn_fdot2(__builtin_bit_cast(sh_h2, w.z), one2, c[sp], false);
                c[sp] = __builtin_amdgcn_fdot2(__builtin_bit_cast(sh_h2, w.w), one2, c[sp], false);
            }
            return (c[0] + c[1]) + (c[2] + c[3]);
        };
        // the block's maximum for this lane's query (lanes r32 and r32 + 32 hold complementary keys), two chains
        auto block_max = [&]() -> float {
            float b0 = -INFINITY, b1 = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) { b0 = fmaxf(b0, sacc[0][r]); b1 = fmaxf(b1, sacc[1][r]); }
            return sh_max_xor32(fmaxf(b0, b1));
        };
        float blk = 0.f, bm = 0.f;
        // m starts at 0; the first block moves it when its maximum is more than kTau away on either side (every
        // block holds a valid key: bm is finite). A later block is tested by its numerators' sum, which the row sum
        // needs anyway: only when some lane's 32 numerators sum past 32 x 2^kTau (so one of them exceeds 2^kTau, and
        // its query's maximum exceeds m by more than kTau) is the maximum formed, and m moves for the queries whose
        // maximum exceeds m by more than kTau, as the first rule would move them.
        bool test;
        if constexpr (first) {
            bm = block_max();
            test = __ballot(fabsf(bm) > kTau) != 0;
        } else {
            blk = psum();
            test = __ballot(blk > 32.f * 256.f) != 0;
            static_assert(kTau == 8.f, "the sum threshold is 32 x 2^kTau");
            if (test) bm = block_max();
        }
        if (test) {                                  // wave-uniform: m may move, O and l rescale, scores again
            const bool move = first ? fabsf(bm) > kTau : bm > kTau;
            const float shift = move ? bm : 0.f;
            // before the first block O and l are still empty: nothing to rescale (2^-shift overflows to +inf for a
            // first-block maximum below -128, and 0 x inf would be NaN)
            if constexpr (!first) {
                const float sc = sh_fast_exp2(-shift);
#pragma unroll
                for (int i = 0; i < DT; ++i) oacc[i] *= sc;
                lsum *= sc;
            }
            mrun += shift;
            set_bias(mrun);
            biased = true;
            scores(stc, sacc, Biased{});
            mask_tail();
            expo();
            if constexpr (!first) blk = psum();
        }
        if constexpr (first) {
            attn_stamp(stamp, last, 3);
            attn_stamp(stamp, last, 4);
            lsum = psum();
        } else {
            lsum += blk;
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            if (j + VA < NJ) vr[(j + VA) % (VA + 1)] = vfrag(j + VA);
            __builtin_amdgcn_sched_barrier(0);       // (the read goes out before this MFMA, not after it)
            if (first && j < DT) oacc[j % DT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vr[j % (VA + 1)], pf[j / DT], sh_f16v{}, 0, 0, 0);
            else oacc[j % DT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vr[j % (VA + 1)], pf[j / DT], oacc[j % DT], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    step(0u, Stage0{}, std::true_type{});            // (S > 0: the host launches no empty sequence)
    for (uint32_t kb = 1; kb < nkb; kb += 2) {
        step(kb, Stage1{}, std::false_type{});
        if (kb + 1 < nkb) step(kb + 1, Stage0{}, std::false_type{});
    }
    sh_wait_vmcnt<0>();      // clamped tail loads land before the LDS is reused below
    __syncthreads();
    attn_stamp(stamp, last, 5);

    const float inv = 1.f / (lsum + __shfl_xor(lsum, 32, 64));   // lanes g = 0, 1 hold complementary keys
    uint16_t *so = (uint16_t *)(smem + 2 * KCH) + wave * (QPW * DH);     // this wave's query rows, now free
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int d0 = 32 * dt + 8 * rb + 4 * g;
            const uint32_t lo = (uint32_t)sh_dev_f2h(oacc[dt][4 * rb] * inv) | ((uint32_t)sh_dev_f2h(oacc[dt][4 * rb + 1] * inv) << 16);
            const uint32_t hi = (uint32_t)sh_dev_f2h(oacc[dt][4 * rb + 2] * inv) | ((uint32_t)sh_dev_f2h(oacc[dt][4 * rb + 3] * inv) << 16);
            const int ch = (d0 >> 3) ^ (r32 & 7);
            *(uint2 *)(so + r32 * DH + ch * 8 + (d0 & 7)) = make_uint2(lo, hi);
        }
    sh_wait_lgkm0();                                 // the wave's own staging is complete
    __builtin_amdgcn_wave_barrier();
    for (int c = lane; c < QPW * DC; c += 64) {
        const int row = c / DC, ch = c % DC;
        const uint32_t qq = qw0 + row;
        if (qq >= S) continue;
        *(uint4 *)(O + (uint64_t)qq * a.ldo + 8 * ch) = ((const uint4 *)so)[row * DC + (ch ^ (row & 7))];
    }
    attn_stamp(stamp, last, 6);
}

// Any dh: one 256-thread block per (query, head, sequence); scores of the row in LDS (S <= 16384).
__global__ __launch_bounds__(256) void k_attn_rows(AttnArgs a) {
    extern __shared__ float sc[];
    __shared__ float red[4];
    const uint32_t qi = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const uint16_t *Q = a.q + b * a.bsq + (uint64_t)h * a.dh + (uint64_t)qi * a.ldq;
    const uint16_t *Kp = a.k + b * a.bsk + (uint64_t)(h / a.grp) * a.dh;
    const uint16_t *Vp = a.v + b * a.bsv + (uint64_t)(h / a.grp) * a.dh;
    uint16_t *O = a.o + b * a.bso + (uint64_t)h * a.dh + (uint64_t)qi * a.ldo;
    // token mask: key j is allowed for query qi iff tok[j] <= tok[qi]; a padding query, or one with no allowed
    // key, averages V uniformly
    const uint32_t tq = a.tok ? a.tok[qi] : 0u;
    bool uni = a.tok && tq == kLlmPad;
    float mx = -INFINITY;
    for (uint32_t j = threadIdx.x; j < a.S; j += 256) {
        float s = 0.f;
        for (uint32_t d = 0; d < a.dh; ++d) s += sh_dev_h2f(Q[d]) * sh_dev_h2f(Kp[(uint64_t)j * a.ldk + d]);
        s *= a.c;
        if (a.tok && a.tok[j] > tq) s = -INFINITY;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = sh_wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    uni = uni || mx == -INFINITY;
    float sum = 0.f;
    for (uint32_t j = threadIdx.x; j < a.S; j += 256) {
        const float p = uni ? 1.f : (sc[j] == -INFINITY ? 0.f : sh_fast_exp2(sc[j] - mx));
        sc[j] = p;
        sum += p;
    }
    sum = sh_wave_sum(sum);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
    __syncthreads();
    const float inv = 1.f / (red[0] + red[1] + red[2] + red[3]);
    for (uint32_t d = threadIdx.x; d < a.dh; d += 256) {
        float acc = 0.f;
        for (uint32_t j = 0; j < a.S; ++j) acc += sc[j] * sh_dev_h2f(Vp[(uint64_t)j * a.ldv + d]);
        O[d] = sh_dev_f2h(acc * inv);
    }
}

// ---- host side ---------------------------------------------------------------------------------------
// stamps: device buffer of 8 s_memrealtime values written by the last stamped launch (see attn_stamp)
struct AttnProfile {
    hipEvent_t e0 = nullptr, e1 = nullptr; bool valid = false; uint32_t entry_ns = 0;
    uint64_t *stamps = nullptr; bool stamped = false;       // stamped: the last launch's kernel wrote the stamps
};
AttnProfile g_prof;

uint32_t l1_bytes_q(uint32_t S, uint32_t dh, uint32_t sq) {     // sh_attention.inc.c:43-51 (uint32 arithmetic)
    const uint32_t kb = S * dh * 2, qb = sq * dh * 2, sb = sq * S * 2;
    return 0x1000u + qb + kb + kb + sb + kb + qb + sq * 4 + 8 * 4;
}

int check_ref(uint32_t S, uint32_t dh, uint32_t sq) {          // sh_attention.inc.c:198-205
    if ((S & 3) || (dh & 3) || sq == 0 || (sq & 3) || S % sq || l1_bytes_q(S, dh, sq) > SH_REF_TCDM_BYTES) {
        sh_set_error(-1, "[sh_attention] S=%u dh=%u sq=%u: need S %% 4 == 0, dh %% 4 == 0, sq | S, sq %% 4 == 0, L1 %u <= %u",
                     S, dh, sq, l1_bytes_q(S, dh, sq ? sq : 1), SH_REF_TCDM_BYTES);
        return -1;
    }
    return 0;
}

// stamp: the launch carries the start / end timestamps sh_attention_profile reports (the reference's entry
// points); the additive batched entry launches without them (no profiling work on the batched hot path).
int run(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t B, uint32_t S, uint32_t dh, uint32_t H,
        uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, uint64_t bsq, uint64_t bsk, uint64_t bsv, uint64_t bso, float scale,
        uint64_t tok = 0, uint32_t grp = 1, bool stamp = true, const uint64_t *pf = nullptr) {
    if (!q || !k || !v || !o) { sh_set_error(-1, "[sh_attention] NULL tensor address"); return -1; }
    if (B == 0 || S == 0 || H == 0 || dh == 0) return 0;
    if (H > 65535 || B > 65535) { sh_set_error(-1, "[sh_attention] H=%u or B=%u above 65535", H, B); return -1; }
    AttnArgs a{(const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)v, (uint16_t *)o,
               ldq, ldk, ldv, ldo, bsq, bsk, bsv, bso, S, dh, scale * 1.4426950408889634f, (const uint16_t *)tok, grp, 1};
    if (pf) {                       // prefetch ranges (address, bytes) x 2 as whole 64-byte lines
        for (int r = 0; r < 2; ++r) {
            if (!pf[2 * r + 1]) continue;
            if (!pf[2 * r]) { sh_set_error(-1, "[sh_attention_batched_prefetch] NULL prefetch address"); return -1; }
            const uint64_t base = pf[2 * r] & ~uint64_t(63), lines = (pf[2 * r] + pf[2 * r + 1] - base + 63) / 64;
            if (lines >= (1ull << 30)) { sh_set_error(-1, "[sh_attention_batched_prefetch] prefetch range above 64 GiB"); return -1; }
            (r ? a.pf1 : a.pf0) = (const uint8_t *)base;
            (r ? a.pfl1 : a.pfl0) = (uint32_t)lines;
        }
    }
    {
        static const int remap = [] { const char *e = getenv("SH_ATTN_XCD"); return (e && *e) ? atoi(e) : 1; }();
        const uint32_t X = (uint32_t)sh_num_xcds();
        const uint64_t gx = sh_cdiv(S, QPB), blocks = gx * H * B, dmax = std::max<uint64_t>(std::max<uint64_t>(X, gx), H);
        if (remap && X > 1 && gx > 1 && ((uint64_t)H * B) % X == 0 && blocks * dmax < (1ull << 32)) {
            auto magic = [](uint64_t d) { return ((1ull << 32) + d - 1) / d; };
            a.xcds = X;
            a.mx = magic(X);
            a.mgx = magic(gx);
            a.mgy = magic(H);
        }
    }
    hipStream_t st = sh_stream();
    if (!g_prof.e0) {
        if (!sh_hip_ok(hipEventCreate(&g_prof.e0), "hipEventCreate") || !sh_hip_ok(hipEventCreate(&g_prof.e1), "hipEventCreate")) return SH_EHIP;
    }
    if (stamp && !g_prof.stamps) {
        hipStreamCaptureStatus cs0 = hipStreamCaptureStatusNone;
        const bool cap0 = hipStreamIsCapturing(st, &cs0) == hipSuccess && cs0 != hipStreamCaptureStatusNone;
        if (!cap0 && !sh_hip_ok(hipMalloc(&g_prof.stamps, 8 * sizeof(uint64_t)), "attention stamps hipMalloc")) return SH_EHIP;
    }
    g_prof.entry_ns = 0;
    // The kernel's start / end timestamps come with its dispatch (no separate event packets on the stream).
    // Under stream capture (a HIP graph) the launch carries no events and the profile is left unset.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    const bool events = stamp && !capturing;
    g_prof.stamped = false;
    auto go = [&](auto kern, dim3 grid, size_t shm) {
        if (!events) hipLaunchKernelGGL(kern, grid, dim3(256), (uint32_t)shm, st, a);
        else hipExtLaunchKernelGGL(kern, grid, dim3(256), (uint32_t)shm, st, g_prof.e0, g_prof.e1, 0u, a);
    };
    // kernels that also write the phase stamps of their last workgroup (only on a stamped, uncaptured call)
    uint64_t *sp = events ? g_prof.stamps : nullptr;
    auto go2 = [&](auto kern, dim3 grid, size_t shm) {
        g_prof.stamped = sp != nullptr;
        if (!events) hipLaunchKernelGGL(kern, grid, dim3(256), (uint32_t)shm, st, a, sp);
        else hipExtLaunchKernelGGL(kern, grid, dim3(256), (uint32_t)shm, st, g_prof.e0, g_prof.e1, 0u, a, sp);
    };
    const bool vec = dh % 8 == 0 && ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0 && ldo % 8 == 0 &&
                     bsq % 8 == 0 && bsk % 8 == 0 && bsv % 8 == 0 && bso % 8 == 0 &&
                     sh_aligned16(q) && sh_aligned16(k) && sh_aligned16(v) && sh_aligned16(o);
    static const int impl = [] { const char *e = getenv("SH_ATTN_IMPL"); return (e && *e) ? atoi(e) : 0; }();
    const dim3 grid(sh_cdiv(S, QPB), H, B);
    const bool fold = fabsf(a.c) <= 1.f;            // c q stays in fp16 range
    if (tok && (dh == 64 || dh == 128) && vec) {
        if (dh == 64) fold ? go2(k_flash2<64, 2, true, true>, grid, 0) : go2(k_flash2<64, 2, true, false>, grid, 0);
        else fold ? go2(k_flash2<128, 2, true, true>, grid, 0) : go2(k_flash2<128, 2, true, false>, grid, 0);
    } else if (tok) {
        if (S > 16384) { sh_set_error(-1, "[sh_attention] masked heads with dh=%u support S <= 16384", dh); return -1; }
        static bool attr_m = false;
        if (!attr_m) { (void)hipFuncSetAttribute((const void *)k_attn_rows, hipFuncAttributeMaxDynamicSharedMemorySize, 16384 * 4); attr_m = true; }
        go(k_attn_rows, dim3(S, H, B), S * sizeof(float));
    } else if ((dh == 64 || dh == 128) && vec && impl != 2 && fold && (uint64_t)KB * (ldk > ldv ? ldk : ldv) * 2 < (1ull << 31)) {
        // (k_flash3 addresses a key block's rows as a scalar base plus 32-bit lane offsets)
        if (a.pfl0 | a.pfl1) {
            if (sp || S % KB != 0) {
                if (dh == 64) sp ? go2(k_flash3<64, 2, true, true>, grid, 0) : go2(k_flash3<64, 2, true, false>, grid, 0);
                else sp ? go2(k_flash3<128, 2, true, true>, grid, 0) : go2(k_flash3<128, 2, true, false>, grid, 0);
            } else {
                if (dh == 64) go2((k_flash3<64, 2, true, false, false>), grid, 0);
                else go2((k_flash3<128, 2, true, false, false>), grid, 0);
            }
            a.pfl0 = a.pfl1 = 0;                    // (this kernel reads the ranges itself: no pass after it)
        } else if (sp || S % KB != 0) {
            if (dh == 64) sp ? go2(k_flash3<64, 2, false, true>, grid, 0) : go2(k_flash3<64, 2, false, false>, grid, 0);
            else sp ? go2(k_flash3<128, 2, false, true>, grid, 0) : go2(k_flash3<128, 2, false, false>, grid, 0);
        } else {                                    // (whole key blocks: the build without the ragged-tail code)
            if (dh == 64) go2((k_flash3<64, 2, false, false, false>), grid, 0);
            else go2((k_flash3<128, 2, false, false, false>), grid, 0);
        }
    } else if ((dh == 64 || dh == 128) && vec) {
        if (dh == 64) fold ? go2(k_flash2<64, 2, false, true>, grid, 0) : go2(k_flash2<64, 2, false, false>, grid, 0);
        else fold ? go2(k_flash2<128, 2, false, true>, grid, 0) : go2(k_flash2<128, 2, false, false>, grid, 0);
    } else if (dh <= 128) {
        if (dh <= 64) {
            if (vec) go(k_flash<64, true>, grid, 0);
            else go(k_flash<64, false>, grid, 0);
        } else {
            if (vec) go(k_flash<128, true>, grid, 0);
            else go(k_flash<128, false>, grid, 0);
        }
    } else {
        if (S > 16384) { sh_set_error(-1, "[sh_attention] dh=%u > 128 supports S <= 16384", dh); return -1; }
        static bool attr = false;
        if (!attr) { (void)hipFuncSetAttribute((const void *)k_attn_rows, hipFuncAttributeMaxDynamicSharedMemorySize, 16384 * 4); attr = true; }
        go(k_attn_rows, dim3(S, H, B), S * sizeof(float));
    }
    if (!sh_launch_ok("sh_attention")) return SH_EHIP;
    if (a.pfl0 | a.pfl1) {                          // a kernel without the prefetch: the same reads after it
        for (int r = 0; r < 2; ++r)
            if (pf[2 * r + 1] && sh_prefetch(pf[2 * r], pf[2 * r + 1]) != 0) return SH_EHIP;
    }
    g_prof.valid = events;         // a batched or captured call leaves no stamps: the profile then reads 0
    return 0;
}

uint32_t q_block_rule(uint32_t S, uint32_t dh, uint32_t H, uint32_t P) {   // sh_attention.inc.c:55-65
    const uint32_t cand[4] = {S, 256, 128, 64};
    uint32_t best = 0, best_rows = 0;
    for (int i = 0; i < 4; ++i) {
        const uint32_t sq = cand[i];
        if (sq == 0 || sq > S || S % sq || sq % 4 || l1_bytes_q(S, dh, sq) > SH_REF_TCDM_BYTES) continue;
        const uint32_t items = H * (S / sq), rows = ((items + P - 1) / P) * sq;
        if (!best || rows < best_rows) { best = sq; best_rows = rows; }
    }
    return best;
}

// The reference's masked head keeps the whole head resident (sh_llm.inc.c:250-272): S <= 256, S % 4, dh % 4,
// scale > 0, and its TCDM (head layout + the token array + one 4-class mask cache per core, 3 cores) must fit.
int check_masked(const char *op, uint32_t S, uint32_t dh, float scale) {
    const uint32_t end = l1_bytes_q(S, dh, S);
    const uint32_t ltok = (end + 63) & ~63u, lcls = ltok + ((S * 2 + 63) & ~63u);
    const uint32_t clsb = (64u + 4u * 2u * S * 2u + 63) & ~63u, lend = lcls + 3u * clsb;
    if (S > 256 || (S & 3) || (dh & 3) || dh == 0 || !(scale > 0.f) || lend > SH_REF_TCDM_BYTES) {
        sh_set_error(-1, "[%s] S=%u dh=%u: need S <= 256, S %% 4 == 0, dh %% 4 == 0, scale > 0, L1 %u <= %u",
                     op, S, dh, lend, SH_REF_TCDM_BYTES);
        return -1;
    }
    return 0;
}

}  // namespace

extern "C" {

uint32_t sh_attention_l1_bytes_q(uint32_t S, uint32_t dh, uint32_t sq) { return l1_bytes_q(S, dh, sq ? sq : S); }
uint32_t sh_attention_l1_bytes(uint32_t S, uint32_t dh) { return sh_attention_l1_bytes_q(S, dh, S); }
uint32_t sh_attention_q_block(uint32_t S, uint32_t dh, uint32_t H, uint32_t P) { return q_block_rule(S, dh, H, P ? P : 1); }

int sh_attention_head(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t dh,
                      uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint32_t) {
    const uint32_t sq = q_block_rule(S, dh, 1, 1);
    if (check_ref(S, dh, sq)) return -1;
    return run(q, k, v, o, 1, S, dh, 1, ldq, ldk, ldv, ldo, 0, 0, 0, 0, scale);
}

int sh_attention_q(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t D, uint32_t H,
                   uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint32_t cluster, uint32_t sq) {
    const uint32_t dh = H ? D / H : 0;
    if (H == 0 || dh * H != D) { sh_set_error(-1, "[sh_attention] D=%u not divisible by H=%u", D, H); return -1; }
    if (!sq) sq = q_block_rule(S, dh, H, cluster == SH_ALL ? 16 : 1);
    if (check_ref(S, dh, sq)) return -1;
    return run(q, k, v, o, 1, S, dh, H, ldq, ldk, ldv, ldo, 0, 0, 0, 0, scale);
}

int sh_attention(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t D, uint32_t H,
                 uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint32_t cluster) {
    return sh_attention_q(q, k, v, o, S, D, H, ldq, ldk, ldv, ldo, scale, cluster, 0);
}

int sh_attention_batched(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t B, uint32_t S, uint32_t D, uint32_t H,
                         uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo,
                         uint64_t bsq, uint64_t bsk, uint64_t bsv, uint64_t bso, float scale, uint32_t sq) {
    const uint32_t dh = H ? D / H : 0;
    if (H == 0 || dh * H != D) { sh_set_error(-1, "[sh_attention_batched] D=%u not divisible by H=%u", D, H); return -1; }
    if (sq && S % sq) { sh_set_error(-1, "[sh_attention_batched] sq=%u does not divide S=%u", sq, S); return -1; }
    return run(q, k, v, o, B, S, dh, H, ldq, ldk, ldv, ldo, bsq, bsk, bsv, bso, scale, 0, 1, false);
}

int sh_attention_batched_prefetch(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t B, uint32_t S, uint32_t D, uint32_t H,
                                  uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo,
                                  uint64_t bsq, uint64_t bsk, uint64_t bsv, uint64_t bso, float scale, uint32_t sq,
                                  uint64_t pf0, uint64_t pf0_bytes, uint64_t pf1, uint64_t pf1_bytes) {
    const uint32_t dh = H ? D / H : 0;
    if (H == 0 || dh * H != D) { sh_set_error(-1, "[sh_attention_batched_prefetch] D=%u not divisible by H=%u", D, H); return -1; }
    if (sq && S % sq) { sh_set_error(-1, "[sh_attention_batched_prefetch] sq=%u does not divide S=%u", sq, S); return -1; }
    const uint64_t pf[4] = {pf0, pf0_bytes, pf1, pf1_bytes};
    return run(q, k, v, o, B, S, dh, H, ldq, ldk, ldv, ldo, bsq, bsk, bsv, bso, scale, 0, 1, false, pf);
}

int sh_attention_head_masked(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t dh,
                             uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint64_t tok, uint32_t) {
    if (check_masked("sh_attention_head_masked", S, dh, scale)) return -1;
    return run(q, k, v, o, 1, S, dh, 1, ldq, ldk, ldv, ldo, 0, 0, 0, 0, scale, tok, 1);
}

int sh_attention_gqa(uint64_t q, uint64_t k, uint64_t v, uint64_t o, uint32_t S, uint32_t D, uint32_t H, uint32_t Hkv,
                     uint32_t ldq, uint32_t ldk, uint32_t ldv, uint32_t ldo, float scale, uint64_t tok, uint32_t) {
    const uint32_t dh = H ? D / H : 0;
    if (H == 0 || Hkv == 0 || dh * H != D || H % Hkv) {                 // sh_llm.inc.c:327-331
        sh_set_error(-1, "[sh_attention_gqa] bad D=%u H=%u Hkv=%u", D, H, Hkv);
        return -1;
    }
    if (check_masked("sh_attention_gqa", S, dh, scale)) return -1;      // every head fails the same way (:333-337)
    return run(q, k, v, o, 1, S, dh, H, ldq, ldk, ldv, ldo, 0, 0, 0, 0, scale, tok, H / Hkv);
}

// ns since the first workgroup of the last stamped launch started (phase 7 = 0): 0 the last workgroup's start,
// 1-2 its operands staged, 3-4 the first key block's scores done (one-pass kernel) or the row maximum known
// (two-pass kernel: pass 1 done), 5 every key block done (P.V), 6 stored. Kernels without stamps report only 6, as the launch's
// event time.
uint32_t sh_attention_profile(uint32_t, uint32_t, uint32_t phase) {
    if (!g_prof.valid) return 0;
    phase &= 7;
    if (hipEventSynchronize(g_prof.e1) != hipSuccess) return 0;
    uint64_t st[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (g_prof.stamped && hipMemcpy(st, g_prof.stamps, sizeof st, hipMemcpyDeviceToHost) == hipSuccess && st[7] && st[6] >= st[7]) {
        return phase == 7 ? 0u : (uint32_t)((st[phase] >= st[7] ? st[phase] - st[7] : 0) * 10u);   // 100 MHz counter
    }
    if (phase != 6) return 0;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, g_prof.e0, g_prof.e1) != hipSuccess) return 0;
    return (uint32_t)((double)ms * 1e6 + 0.5);
}

}  // extern "C"
