// Runtime services behind the reference's wrapper functions (reference runtime/sh_rt.inc.c:2-59):
// device/stream state, the HBM arena behind sh_hbm_addr, HIP-event timers, printf capture, error state,
// the library workspace, and the host IEEE binary16 codec.
#include "sh_common.h"
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <map>
#include <vector>

namespace {
struct ShState {
    bool init = false;
    int device = 0;
    int cus = 0;
    int xcds = 1;
    hipStream_t stream = nullptr;          // nullptr = legacy null stream
    void *arena = nullptr;
    size_t arena_bytes = 0;
    std::vector<void *> mallocs;
    // split-K partial workspaces, one per stream (calls on different streams never share partials); an outgrown
    // buffer is retired, not freed, because a HIP graph captured earlier may still address it. Everything a stream
    // holds is freed by sh_stream_release.
    struct Ws { void *p = nullptr; size_t bytes = 0; std::vector<void *> retired; };
    std::map<hipStream_t, Ws> ws;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    bool timer_running = false;
    double last_ns = 0.0;
    std::chrono::steady_clock::time_point t0;
    int last_err = 0;
    std::string last_msg;
    bool capture = false;
    std::string captured;
    uint32_t eoc = 0;
};
ShState g;
}  // namespace

static void sh_out(const char *s) {
    if (g.capture) g.captured += s;
    else { fputs(s, stdout); fflush(stdout); }
}

void sh_set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list va; va_start(va, fmt);
    vsnprintf(buf, sizeof buf, fmt, va);
    va_end(va);
    g.last_err = code;
    g.last_msg = buf;
    fprintf(stderr, "%s\n", buf);
    fflush(stderr);
}

bool sh_hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    sh_set_error(SH_EHIP, "[softhier-ops] %s: %s", what, hipGetErrorString(e));
    return false;
}

bool sh_launch_ok(const char *what) { return sh_hip_ok(hipGetLastError(), what); }

void sh_ensure_init() { if (!g.init) sh_init(); }
hipStream_t sh_stream() { sh_ensure_init(); return g.stream; }
int sh_num_cus() { sh_ensure_init(); return g.cus; }
int sh_num_xcds() { sh_ensure_init(); return g.xcds; }

void *sh_workspace(size_t bytes) {
    sh_ensure_init();
    ShState::Ws &w = g.ws[g.stream];
    if (bytes <= w.bytes) return w.p;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g.stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        sh_set_error(SH_EHIP, "[softhier-ops] split-K workspace of %zu B needed under stream capture (this stream holds %zu B): "
                     "run the call once on this stream before capturing it", bytes, w.bytes);
        return nullptr;
    }
    // geometric growth keeps the retired buffers below the live one in total
    size_t want = bytes < (size_t(64) << 20) ? (size_t(64) << 20) : bytes;
    if (want < 2 * w.bytes) want = 2 * w.bytes;
    void *p = nullptr;
    if (!sh_hip_ok(hipMalloc(&p, want), "workspace hipMalloc")) return nullptr;
    if (w.p) w.retired.push_back(w.p);
    w.p = p;
    w.bytes = want;
    return w.p;
}

extern "C" {

void sh_init(void) {
    if (g.init) return;
    g.init = true;
    g.t0 = std::chrono::steady_clock::now();
    if (!sh_hip_ok(hipGetDevice(&g.device), "hipGetDevice")) return;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, g.device) == hipSuccess) g.cus = v;
    v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, g.device) == hipSuccess && v > 0) g.xcds = v;
    sh_hip_ok(hipEventCreate(&g.ev0), "hipEventCreate");
    sh_hip_ok(hipEventCreate(&g.ev1), "hipEventCreate");
}

int sh_stream_release(uint64_t stream) {
    sh_ensure_init();
    const hipStream_t st = (hipStream_t)stream;
    auto it = g.ws.find(st);
    if (it == g.ws.end()) return 0;
    if (!sh_hip_ok(hipStreamSynchronize(st), "sh_stream_release hipStreamSynchronize")) return SH_EHIP;
    int rc = 0;
    if (it->second.p && !sh_hip_ok(hipFree(it->second.p), "sh_stream_release hipFree")) rc = SH_EHIP;
    for (void *p : it->second.retired)
        if (!sh_hip_ok(hipFree(p), "sh_stream_release hipFree")) rc = SH_EHIP;
    g.ws.erase(it);
    return rc;
}

uint64_t sh_stream_workspace_bytes(uint64_t stream) {
    auto it = g.ws.find((hipStream_t)stream);
    if (it == g.ws.end()) return 0;
    return it->second.bytes;
}

void sh_barrier_global(void) { sh_ensure_init(); sh_hip_ok(hipStreamSynchronize(g.stream), "sh_barrier_global"); }
void sh_barrier_cluster(void) { sh_barrier_global(); }
uint32_t sh_cluster_id(void) { return 0; }
uint32_t sh_core_id(void) { return 0; }
int sh_is_first_core(void) { return 1; }
int sh_is_dm_core(void) { return 1; }
uint32_t sh_num_clusters(void) { return 1; }
uint32_t sh_l1_size(void) { return SH_REF_TCDM_BYTES; }

void sh_timer_start(void) {
    sh_ensure_init();
    if (sh_hip_ok(hipEventRecord(g.ev0, g.stream), "sh_timer_start")) g.timer_running = true;
}

void sh_timer_end(void) {
    sh_ensure_init();
    if (!g.timer_running) return;
    if (!sh_hip_ok(hipEventRecord(g.ev1, g.stream), "sh_timer_end")) return;
    if (!sh_hip_ok(hipEventSynchronize(g.ev1), "sh_timer_end sync")) return;
    float ms = 0.f;
    if (!sh_hip_ok(hipEventElapsedTime(&ms, g.ev0, g.ev1), "sh_timer_end elapsed")) return;
    g.last_ns = (double)ms * 1e6;
    char buf[128];
    snprintf(buf, sizeof buf, "[Performance Counter]: Execution period is %llu ns\n", (unsigned long long)(g.last_ns + 0.5));
    sh_out(buf);
    sh_hip_ok(hipEventRecord(g.ev0, g.stream), "sh_timer_end restart");   // the next ROI starts here
}

double sh_timer_last_ns(void) { return g.last_ns; }

void sh_eoc(uint32_t val) {
    sh_barrier_global();
    g.eoc = val;
    fflush(stdout);
}

uint32_t sh_cycles(void) {
    sh_barrier_global();
    auto d = std::chrono::steady_clock::now() - g.t0;
    return (uint32_t)std::chrono::duration_cast<std::chrono::nanoseconds>(d).count();
}

void sh_printf(const char *fmt, ...) {
    char small[512];
    va_list va, vb;
    va_start(va, fmt);
    va_copy(vb, va);
    const int n = vsnprintf(small, sizeof small, fmt, va);
    va_end(va);
    if (n >= 0 && (size_t)n >= sizeof small) {      // long text (sample dumps): format again at full length
        std::string big((size_t)n + 1, '\0');
        vsnprintf(&big[0], big.size(), fmt, vb);
        big.resize((size_t)n);
        sh_out(big.c_str());
    } else if (n >= 0) {
        sh_out(small);
    }
    va_end(vb);
}

uint64_t sh_hbm_addr(uint64_t off) {
    sh_ensure_init();
    if (!g.arena) {
        size_t bytes = size_t(1) << 30;
        if (const char *e = getenv("SH_HBM_ARENA_BYTES")) {
            unsigned long long v = strtoull(e, nullptr, 0);
            if (v) bytes = (size_t)v;
        }
        if (!sh_hip_ok(hipMalloc(&g.arena, bytes), "HBM arena hipMalloc")) { g.arena = nullptr; return 0; }
        if (!sh_hip_ok(hipMemset(g.arena, 0, bytes), "HBM arena clear")) return 0;
        g.arena_bytes = bytes;
    }
    if (off >= g.arena_bytes) {
        sh_set_error(-1, "[sh_hbm_addr] offset 0x%llx beyond the %llu B arena (SH_HBM_ARENA_BYTES)",
                     (unsigned long long)off, (unsigned long long)g.arena_bytes);
        return 0;
    }
    return (uint64_t)(uintptr_t)g.arena + off;
}

uint64_t sh_hbm_malloc(uint32_t bytes) {
    sh_ensure_init();
    void *p = nullptr;
    if (!sh_hip_ok(hipMalloc(&p, bytes ? bytes : 1), "sh_hbm_malloc")) return 0;
    g.mallocs.push_back(p);
    return (uint64_t)(uintptr_t)p;
}

void sh_preload_wait(uint64_t) { sh_barrier_global(); }

// Preload image (reference softhier_mlir/sim/preload.py:38-78): an ELF32 whose PT_LOAD segments place data at
// physical address SH_PRELOAD_HBM_BASE + offset. Every segment is copied into the arena at that offset, so the
// program's sh_hbm_addr(offset) buffers hold it; the file is checked completely before the first copy.
int sh_preload_load(const char *path) {
    if (!path) { sh_set_error(-1, "[sh_preload_load] NULL path"); return -1; }
    FILE *f = fopen(path, "rb");
    if (!f) { sh_set_error(-1, "[sh_preload_load] cannot open %s", path); return -1; }
    std::vector<uint8_t> img;
    uint8_t buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) img.insert(img.end(), buf, buf + n);
    fclose(f);
    auto u16 = [&](size_t o) { uint16_t v; memcpy(&v, &img[o], 2); return v; };
    auto u32 = [&](size_t o) { uint32_t v; memcpy(&v, &img[o], 4); return v; };
    if (img.size() < 52 || memcmp(img.data(), "\x7f" "ELF", 4) != 0 || img[4] != 1 || img[5] != 1) {
        sh_set_error(-1, "[sh_preload_load] %s is not a little-endian ELF32 image", path);
        return -1;
    }
    const size_t phoff = u32(28), phentsize = u16(42), phnum = u16(44);
    if (phentsize < 32 || phoff + phnum * phentsize > img.size()) {
        sh_set_error(-1, "[sh_preload_load] %s: program headers outside the file", path);
        return -1;
    }
    struct Seg { uint64_t off; size_t file_off, bytes; };
    std::vector<Seg> segs;
    for (size_t i = 0; i < phnum; ++i) {
        const size_t h = phoff + i * phentsize;
        if (u32(h) != 1) continue;                                   // PT_LOAD only
        const size_t fo = u32(h + 4), bytes = u32(h + 16);
        const uint64_t paddr = u32(h + 12);
        if (fo + bytes > img.size() || paddr < SH_PRELOAD_HBM_BASE) {
            sh_set_error(-1, "[sh_preload_load] %s: segment %zu outside the file or below the HBM base", path, i);
            return -1;
        }
        segs.push_back({paddr - SH_PRELOAD_HBM_BASE, fo, bytes});
    }
    if (!sh_hbm_addr(0)) return SH_EHIP;                           // the arena exists (allocated, zeroed)
    for (const Seg &sg : segs)
        if (sg.off + sg.bytes > g.arena_bytes) {
            sh_set_error(-1, "[sh_preload_load] %s: segment at 0x%llx (+%zu B) beyond the %llu B arena (SH_HBM_ARENA_BYTES)", path,
                         (unsigned long long)sg.off, sg.bytes, (unsigned long long)g.arena_bytes);
            return -1;
        }
    sh_barrier_global();                                           // nothing queued still reads or writes the arena
    for (const Seg &sg : segs)
        if (sg.bytes && !sh_hip_ok(hipMemcpy((char *)g.arena + sg.off, img.data() + sg.file_off, sg.bytes, hipMemcpyHostToDevice),
                                   "sh_preload_load copy"))
            return SH_EHIP;
    return (int)segs.size();
}

void sh_call_on_core_stack(void (*fn)(void), uint32_t) { if (fn) fn(); }

int sh_last_error(void) { int e = g.last_err; g.last_err = 0; return e; }
const char *sh_last_error_str(void) { return g.last_msg.c_str(); }
void sh_set_stream(uint64_t s) { sh_ensure_init(); g.stream = (hipStream_t)(uintptr_t)s; }
uint64_t sh_get_stream(void) { sh_ensure_init(); return (uint64_t)(uintptr_t)g.stream; }

void sh_capture(int on) { g.capture = on != 0; if (on) g.captured.clear(); }
uint64_t sh_captured(char *buf, uint64_t cap) {
    const uint64_t n = g.captured.size();
    if (buf && cap) {
        const uint64_t m = n < cap - 1 ? n : cap - 1;
        memcpy(buf, g.captured.data(), m);
        buf[m] = 0;
    }
    return n;
}

// IEEE 754 binary16 <-> binary32 (host). binary16: 1 sign, 5 exponent (bias 15), 10 fraction bits.
float sh_fp16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1Fu, fr = h & 0x3FFu;
    uint32_t bits;
    if (ex == 0x1F) {
        bits = sign | 0x7F800000u | (fr << 13);                 // Inf / NaN (payload kept)
    } else if (ex != 0) {
        bits = sign | ((ex + 127 - 15) << 23) | (fr << 13);      // normal
    } else if (fr == 0) {
        bits = sign;                                             // signed zero
    } else {                                                     // subnormal: fr * 2^-24, normalise
        int shift = 0;
        uint32_t f = fr;
        while (!(f & 0x400u)) { f <<= 1; ++shift; }
        bits = sign | ((uint32_t)(127 - 14 - shift) << 23) | ((f & 0x3FFu) << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

uint16_t sh_f32_to_fp16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t ex = (u >> 23) & 0xFFu, fr = u & 0x7FFFFFu;
    if (ex == 0xFF) return (uint16_t)(sign | (fr ? 0x7E00u : 0x7C00u));   // NaN -> quiet canonical, Inf
    const int e = (int)ex - 127;                                        // unbiased exponent
    if (e > 15) return (uint16_t)(sign | 0x7C00u);                      // overflow before rounding
    // value = 1.fr * 2^e (normal f32) ; binary16 keeps 10 fraction bits down to 2^-14, then 2^-24 steps
    uint32_t mant = fr | 0x800000u;                                     // 24-bit significand
    if (ex == 0) return sign;                                           // f32 subnormals are < 2^-126: zero
    int drop;                                                           // low bits of `mant` to discard
    uint32_t base;                                                      // result bits before the significand
    if (e >= -14) { drop = 13; base = (uint32_t)(e + 15) << 10; mant &= 0x7FFFFFu; mant |= 0x800000u; }
    else {
        drop = 13 + (-14 - e);                                          // subnormal result
        if (drop > 24) return sign;                                     // below half the smallest subnormal
        base = 0;
    }
    uint32_t q = mant >> drop;
    const uint32_t rem = mant & ((1u << drop) - 1), half = 1u << (drop - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;                   // round to nearest, ties to even
    uint32_t r;
    if (e >= -14) r = base + (q - 0x400u);                              // drop the implicit bit; a carry bumps the exponent
    else r = q;                                                         // may round up into the smallest normal
    if (r >= 0x7C00u) r = 0x7C00u;                                      // rounded up to Inf
    return (uint16_t)(sign | r);
}

}  // extern "C"
