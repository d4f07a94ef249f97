// Internal declarations shared by the softhier-ops HIP sources (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include "sh_ops.h"

typedef _Float16 sh_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 sh_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 sh_h2 __attribute__((ext_vector_type(2)));
typedef float sh_f16v __attribute__((ext_vector_type(16)));
typedef float sh_f4v __attribute__((ext_vector_type(4)));

// The reference cluster's TCDM bytes (ARCH_CLUSTER_TCDM_SIZE, softhier_mlir/sim/gvsoc.py:56): every
// budget check the reference makes is made against this number so calls fail here exactly when they fail there.
#define SH_REF_TCDM_BYTES 0x100000u

// ---- runtime services (sh_rt.hip) -------------------------------------------------------------------
hipStream_t sh_stream();                       // the library stream (after sh_init)
void sh_ensure_init();                         // sh_init() on first use
int sh_num_cus();                              // compute units of the current device
int sh_num_xcds();                             // XCDs (8 on MI355X); dispatch is round-robin over them
// Record a failure: prints "[tag] message" on stderr once per call site and sets sh_last_error.
void sh_set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Check a HIP call; on failure records SH_EHIP and returns false.
bool sh_hip_ok(hipError_t e, const char *what);
// Check the last kernel launch.
bool sh_launch_ok(const char *what);
// Library-owned device workspace of at least `bytes` for the library stream: one buffer per stream, grown on
// demand (never under stream capture: that is an error), outgrown buffers kept until the process ends.
void *sh_workspace(size_t bytes);

// ---- device helpers ---------------------------------------------------------------------------------
__device__ __forceinline__ float sh_dev_h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t sh_dev_f2h(float f) {   // v_cvt_f16_f32: round to nearest even
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// The same for a value that must be rounded to fp32 first: without the empty asm the compiler may fold the
// conversion into the fp32 multiply-add that produced the value (v_fma_mix*, one rounding instead of two) in one
// build and not in another, and two kernels would then store different bits for the same operands.
__device__ __forceinline__ uint16_t sh_dev_f2h_rr(float f) {
    asm volatile("" : "+v"(f));
    return sh_dev_f2h(f);
}
// Correctly rounded fp16 addition of packed pairs (v_pk_add_f16, round to nearest even). For fp16 operands
// this equals rounding their fp32 sum to fp16: fp32 keeps 24 >= 2*11 + 2 significand bits, which makes the
// double rounding exact (Figueroa, "When is double rounding innocuous?", SIGNUM 1995).
__device__ __forceinline__ uint32_t sh_hadd2(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(sh_h2, a) + __builtin_bit_cast(sh_h2, b));
}
__device__ __forceinline__ float sh_fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float sh_fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float sh_fast_rsq(float x) { return __builtin_amdgcn_rsqf(x); }

// tanh-form GELU: 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3), written as x / (1 + e^{-2u})
// = x / (1 + 2^{x (k0 + k1 x^2)}) with k0 = -2 sqrt(2/pi) log2(e), k1 = 0.044715 k0, evaluated on fp16 pairs
// (packed fp16 multiply / fma / add, hardware fp16 exp2 and reciprocal): 3.5 VALU + 2 transcendental
// instructions per element. Relative error is a few fp16 ulps where the result is not negligible. Overflow
// needs no clamp: 2^t = inf gives x * rcp(inf) = 0, 2^t = 0 gives x. Every caller (row op, GEMM epilogue,
// split-K reduction) uses this one function, so fused and unfused sequences store identical bits: each step
// rounds to fp16 as written, which leaves the compiler no product to fuse with a later rounding (an fp32 form,
// x * rcp(1 + e) in fp32 and then fp16, was compiled into a single-rounding fp16 fma in one kernel and two
// roundings in another).
#define SH_GELU_K0 (-2.3022082f)
#define SH_GELU_K1 (-0.10294324f)
__device__ __forceinline__ sh_h2 sh_gelu_h2(sh_h2 x) {
#pragma clang fp contract(off)
    const sh_h2 k0 = {(_Float16)SH_GELU_K0, (_Float16)SH_GELU_K0}, k1 = {(_Float16)SH_GELU_K1, (_Float16)SH_GELU_K1};
    const sh_h2 t = __builtin_elementwise_fma(x * x, k1, k0) * x;
    const sh_h2 e = {__builtin_elementwise_exp2(t.x), __builtin_elementwise_exp2(t.y)};
    const sh_h2 d = e + (sh_h2){(_Float16)1.0f, (_Float16)1.0f};
    const sh_h2 r = {(_Float16)__builtin_amdgcn_rcph(d.x), (_Float16)__builtin_amdgcn_rcph(d.y)};
    return x * r;
}
__device__ __forceinline__ uint32_t sh_gelu_u32(uint32_t pair) {   // two fp16 codes in a 32-bit word
    return __builtin_bit_cast(uint32_t, sh_gelu_h2(__builtin_bit_cast(sh_h2, pair)));
}

__device__ __forceinline__ float sh_wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float sh_wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// ---- global -> LDS DMA and LDS transpose reads (GEMM and attention kernels) ----------------------------
// One global_load_lds_dwordx4: each lane's 16 bytes at `src` land in LDS at lds_wave_base + 16 * lane (M0 holds
// the wave's LDS base). Completion is counted by vmcnt like any vector memory load.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void sh_lds_dma16(const void *src, uint32_t lds_wave_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_wave_base), "v"(src) : "memory", "m0");
}
// The same with the address split into a wave-uniform base (a scalar register pair) and each lane's 32-bit byte
// offset from it: no 64-bit per-lane address arithmetic.
__device__ __forceinline__ void sh_lds_dma16_s(const void *base, uint32_t off, uint32_t lds_wave_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_wave_base), "v"(off), "s"(base) : "memory", "m0");
}
#pragma clang diagnostic pop

// The larger of v in lanes l and l ^ 32, in every lane: one v_permlane32_swap of v with itself puts each lane's
// partner value in one of the two results and its own in the other (no LDS round trip).
__device__ __forceinline__ float sh_max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt left unconstrained (gfx9 encoding: vmcnt[3:0], [15:14]).
template <int N>
__device__ __forceinline__ void sh_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// s_waitcnt lgkmcnt(0) with vmcnt / expcnt left unconstrained.
__device__ __forceinline__ void sh_wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Byte address of a __shared__ object in the LDS aperture.
__device__ __forceinline__ uint32_t sh_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// ds_read_b64_tr_b16: in a group of 16 lanes, lane i supplies the address of an 8-byte segment (4 halves) that
// is row i / 4, columns 4 (i % 4) .. 4 (i % 4) + 3 of a 4 x 16 block of halves; lane i receives column i of that
// block (its 4 halves, rows 0..3).
typedef short sh_s4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ sh_s4 sh_ds_read_tr(uint32_t addr) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) sh_s4 *)(uintptr_t)addr);
}

static inline bool sh_aligned16(uint64_t p) { return (p & 15u) == 0; }
static inline uint32_t sh_cdiv(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Division of a 32-bit index by a runtime-invariant divisor d >= 1 with one multiply-high (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994, fig. 4.1): with l = ceil(log2 d)
// and m = floor(2^32 (2^l - d) / d) + 1, n / d = (t + ((n - t) >> 1)) >> (l - 1), t = mulhi(m, n), l >= 1.
struct ShDiv { uint32_t d, mul, l; };
static inline ShDiv sh_make_div(uint32_t d) {
    ShDiv f{d, 0, 0};
    if (d <= 1) return f;
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    f.l = l;
    f.mul = (uint32_t)((((1ull << l) - d) << 32) / d + 1);
    return f;
}
__device__ __forceinline__ uint32_t sh_div(uint32_t n, ShDiv f) {
    if (f.d <= 1) return n;
    const uint32_t t = __umulhi(n, f.mul);
    return (t + ((n - t) >> 1)) >> (f.l - 1);
}
