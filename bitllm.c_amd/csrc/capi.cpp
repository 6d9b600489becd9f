// capi.cpp -- the host-pointer drop-in ABI (eif_quantize_bitnet.h, eif_gemm.h, eif_quant_linear.h) over the
// device kernels, plus device selection and the WHT norm helper of eif_hip.h.
//
// Calling convention kept from the reference (src/eif_quantize_bitnet.c, src/eif_gemm.c): host pointers,
// synchronous return, NULL scales = 1, NULL bias = 0, invalid sizes are a silent no-op. Re-entrancy: the
// reference engines call these symbols from OpenMP worker threads (src/eif_tinyllm.c:1020,
// src/eif_qwen35.c:139-140), so every thread owns its stream and staging buffers; the resident-weight cache is
// shared under a mutex. Weight bytes (and the block scales of eif_matmul_bitnet_block_f32) are uploaded once per
// (host pointer, size, format) and kept in the device layout the kernels read -- the reference's weights live in
// long-lived pools or mmaps (src/eif_tinyllm.c:2565-2731, src/eif_qwen35.c:1229); a caller that rewrites a
// buffer in place calls eif_hip_forget_host_weights(). GEMM operands are never cached (qwen35
// dequantizes into reused temporaries, src/eif_qwen35.c:1038-1049).
//
// There is no CPU fallback: without a gfx950 device every compute entry point prints why and aborts, or, in the
// record error mode (eif_hip_set_host_error_mode), returns and records the error for the calling thread.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <memory>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#include "hip_common.h"
#include "../../include/eif_gemm.h"
#include "../../include/eif_gpu_bitnet.h"
#include "../../include/eif_quant_linear.h"
#include "../../include/eif_quantize_bitnet.h"

namespace {

struct DevState {
    bool ok = false;
    int device = 0;
    std::string why;
};

DevState &dev_state()
{
    static DevState st;
    static std::once_flag once;
    std::call_once(once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
            st.why = "no HIP device visible";
            return;
        }
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, 0) != hipSuccess) {
            st.why = "hipGetDeviceProperties failed";
            return;
        }
        if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
            st.why = std::string("device 0 is ") + p.gcnArchName + ", this library is built for gfx950 only";
            return;
        }
        st.ok = true;
    });
    return st;
}

// Error policy (eif_hip_set_host_error_mode): abort, or record the error for the calling thread and end the call.
// In record mode die() throws HostError, which each entry point catches (a function-try-block) and returns from;
// the lock guards on the way release their mutexes.
std::atomic<int> g_host_err_mode{EIF_HIP_HOST_ABORT};
thread_local int t_err_code = EIF_HIP_OK;
thread_local char t_err_msg[256];
thread_local int t_force_record = 0;   // > 0: record whatever the global mode (the GPU seat's bool contract)
struct HostError {};

// Record mode for the calling thread while it lives, whatever eif_hip_set_host_error_mode says.
struct ForceRecord {
    ForceRecord() { ++t_force_record; }
    ~ForceRecord() { --t_force_record; }
};

[[noreturn]] void die(const char *fn, const char *what)
{
    if (t_force_record > 0 || g_host_err_mode.load(std::memory_order_relaxed) == EIF_HIP_HOST_RECORD) {
        t_err_code = EIF_HIP_E_DEVICE;
        snprintf(t_err_msg, sizeof t_err_msg, "%s: %s", fn, what);
        throw HostError{};
    }
    fprintf(stderr, "libbitllm_hip: %s: %s (no CPU fallback exists)\n", fn, what);
    fflush(stderr);
    abort();
}

#define DIE_ON(expr, fn)                                                  \
    do {                                                                  \
        hipError_t e__ = (expr);                                          \
        if (e__ != hipSuccess) die(fn, hipGetErrorString(e__));           \
    } while (0)

#define DIE_RC(expr, fn)                                                  \
    do {                                                                  \
        int rc__ = (expr);                                                \
        if (rc__ != EIF_HIP_OK) die(fn, eif_hip_strerror(rc__));          \
    } while (0)

// Per-thread stream and growable staging buffers (slots). Never freed: threads of the reference engines live
// for the process, and freeing at thread exit could run after the HIP runtime has shut down.
struct ThreadCtx {
    hipStream_t st = nullptr;
    void *buf[8] = {};
    size_t cap[8] = {};
    // pinned host bounce buffers of the uploads (per slot) and of the download: a copy from or to pageable memory
    // would otherwise be staged by the runtime on every call
    void *pin[9] = {};
    size_t pcap[9] = {};
    bool pending = false;   // an upload from a pinned buffer may still be in flight (no download has synced since)
};
thread_local ThreadCtx t_ctx;

ThreadCtx &ctx(const char *fn)
{
    DevState &d = dev_state();
    if (!d.ok) die(fn, d.why.c_str());
    if (!t_ctx.st) {
        DIE_ON(hipSetDevice(d.device), fn);
        DIE_ON(hipStreamCreateWithFlags(&t_ctx.st, hipStreamNonBlocking), fn);
    }
    return t_ctx;
}

// The calling thread's context at the start of a host-ABI call. A previous call that ended before its download
// (an error in record mode) may still have copies in flight from the pinned buffers, so the stream is drained
// once here. The uploads of one call use distinct pinned buffers, so they never wait for each other.
ThreadCtx &call_ctx(const char *fn)
{
    ThreadCtx &c = ctx(fn);
    if (c.pending) {
        DIE_ON(hipStreamSynchronize(c.st), fn);
        c.pending = false;
    }
    return c;
}

// Device memory owned until released: frees itself on the error paths of record mode (die() throws).
struct DevBuf {
    void *p = nullptr;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    ~DevBuf()
    {
        if (p) (void)hipFree(p);
    }
    void *release()
    {
        void *q = p;
        p = nullptr;
        return q;
    }
};

void *slot(ThreadCtx &c, int i, size_t bytes, const char *fn)
{
    if (bytes == 0) bytes = 16;
    if (c.cap[i] < bytes) {
        if (c.buf[i]) {
            DIE_ON(hipStreamSynchronize(c.st), fn);
            DIE_ON(hipFree(c.buf[i]), fn);
        }
        size_t cap = bytes + bytes / 4 + 256;
        DIE_ON(hipMalloc(&c.buf[i], cap), fn);
        c.cap[i] = cap;
    }
    return c.buf[i];
}

// Pinned bounce buffer i (0..7 uploads, 8 the download) of at least `bytes`, or nullptr above kPinMax (the copy then
// goes from the caller's memory directly). Grown buffers are freed after the stream has drained.
constexpr size_t kPinMax = (size_t)4 << 20;

void *pinned(ThreadCtx &c, int i, size_t bytes, const char *fn)
{
    if (bytes > kPinMax) return nullptr;
    if (c.pcap[i] < bytes) {
        if (c.pin[i]) {
            DIE_ON(hipStreamSynchronize(c.st), fn);
            c.pending = false;
            DIE_ON(hipHostFree(c.pin[i]), fn);
            c.pin[i] = nullptr;
            c.pcap[i] = 0;
        }
        const size_t cap = std::max<size_t>(bytes + bytes / 4, 4096);
        DIE_ON(hipHostMalloc(&c.pin[i], cap, hipHostMallocDefault), fn);
        c.pcap[i] = cap;
    }
    return c.pin[i];
}

void *upload(ThreadCtx &c, int i, const void *host, size_t bytes, const char *fn)
{
    if (!host) return nullptr;
    void *d = slot(c, i, bytes, fn);
    void *p = pinned(c, i, bytes, fn);
    if (p) {
        std::memcpy(p, host, bytes);
        DIE_ON(hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, c.st), fn);
        c.pending = true;
    } else {
        DIE_ON(hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, c.st), fn);
    }
    return d;
}

// A kernel's output buffer: the pinned download buffer itself (the device writes it over PCIe, so no copy follows
// the kernel), or device slot i above kPinMax.
void *out_slot(ThreadCtx &c, int i, size_t bytes, const char *fn)
{
    void *p = pinned(c, 8, bytes, fn);
    return p ? p : slot(c, i, bytes, fn);
}

void download_sync(ThreadCtx &c, void *host, const void *dev, size_t bytes, const char *fn)
{
    if (dev == c.pin[8]) {   // written in place by the kernel
        DIE_ON(hipStreamSynchronize(c.st), fn);
        c.pending = false;
        std::memcpy(host, dev, bytes);
        return;
    }
    void *p = pinned(c, 8, bytes, fn);
    DIE_ON(hipMemcpyAsync(p ? p : host, dev, bytes, hipMemcpyDeviceToHost, c.st), fn);
    DIE_ON(hipStreamSynchronize(c.st), fn);
    c.pending = false;
    if (p) std::memcpy(host, p, bytes);
}

// ---- resident weights ----
enum Kind { kRaw = 0, kQTernRow = 1, kBlockScales = 2, kTiles = 3 };   // kTiles + a reference layout (eif::kSrc*)

struct WKey {
    const void *p;
    size_t n;
    int kind, rows, cols;
    bool operator==(const WKey &o) const
    {
        return p == o.p && n == o.n && kind == o.kind && rows == o.rows && cols == o.cols;
    }
};
struct WKeyHash {
    size_t operator()(const WKey &k) const
    {
        return std::hash<const void *>()(k.p) ^ (k.n * 0x9E3779B97F4A7C15ull) ^ ((size_t)k.kind << 56) ^
               ((size_t)k.rows << 20) ^ (size_t)k.cols;
    }
};
struct WEntry {
    void *raw = nullptr;
    eif_hip_qweight *q = nullptr;
    size_t bytes = 0;     // device bytes held
    int pins = 0;         // calls using it now
    uint64_t used = 0;    // last use (g_tick)
};

// The resident copies are bounded: an insertion beyond the limit evicts the least recently used copies that no
// call is using (every call synchronizes with its stream before it unpins, so an unpinned copy has no work in
// flight). A call pins what it looks up until it returns (PinScope).
std::mutex g_wmu;
std::unordered_map<WKey, WEntry, WKeyHash> g_wcache;
size_t g_cache_bytes = 0, g_cache_limit = 0;   // limit 0: three quarters of the device's memory
uint64_t g_tick = 0;
thread_local std::vector<WKey> t_pins;

void free_entry(const WEntry &e)
{
    if (e.raw) (void)hipFree(e.raw);
    if (e.q) eif_hip_qweight_destroy(e.q);
}

size_t cache_limit()   // g_wmu held
{
    if (g_cache_limit) return g_cache_limit;
    size_t free_b = 0, total = 0;
    if (hipMemGetInfo(&free_b, &total) != hipSuccess || total == 0) return SIZE_MAX;
    return total / 4 * 3;
}

void make_room(size_t need)   // g_wmu held
{
    const size_t lim = cache_limit();
    while (g_cache_bytes + need > lim) {
        auto victim = g_wcache.end();
        for (auto it = g_wcache.begin(); it != g_wcache.end(); ++it)
            if (it->second.pins == 0 && (victim == g_wcache.end() || it->second.used < victim->second.used)) victim = it;
        if (victim == g_wcache.end()) return;   // everything is in use: exceed the limit rather than fail
        g_cache_bytes -= victim->second.bytes;
        free_entry(victim->second);
        g_wcache.erase(victim);
    }
}

WEntry &pin(const WKey &k, WEntry &e)   // g_wmu held
{
    ++e.pins;
    e.used = ++g_tick;
    t_pins.push_back(k);
    return e;
}

WEntry &insert(const WKey &k, const WEntry &e)   // g_wmu held
{
    g_cache_bytes += e.bytes;
    return pin(k, g_wcache.emplace(k, e).first->second);
}

struct PinScope {
    ~PinScope()
    {
        if (t_pins.empty()) return;
        std::lock_guard<std::mutex> lock(g_wmu);
        for (const WKey &k : t_pins) {
            auto it = g_wcache.find(k);
            if (it != g_wcache.end() && it->second.pins > 0) --it->second.pins;
        }
        t_pins.clear();
    }
};

const void *resident_raw(const void *host, size_t n, const char *fn)
{
    ThreadCtx &c = ctx(fn);
    WKey k{host, n, kRaw, 0, 0};
    std::lock_guard<std::mutex> lock(g_wmu);
    auto it = g_wcache.find(k);
    if (it != g_wcache.end()) return pin(k, it->second).raw;
    WEntry e;
    e.bytes = n ? n : 16;
    make_room(e.bytes);
    DevBuf raw;
    DIE_ON(hipMalloc(&raw.p, e.bytes), fn);
    DIE_ON(hipMemcpyAsync(raw.p, host, n, hipMemcpyHostToDevice, c.st), fn);
    DIE_ON(hipStreamSynchronize(c.st), fn);
    e.raw = raw.release();
    return insert(k, e).raw;
}

// The row-tile copy (f32linear.hip) of a weight buffer in reference layout src_fmt (n bytes): the bytes go up once,
// are repacked on the device and dropped.
const void *resident_tiles(const void *host, size_t n, int src_fmt, int rows, int cols, const char *fn)
{
    ThreadCtx &c = ctx(fn);
    WKey k{host, n, kTiles + src_fmt, rows, cols};
    std::lock_guard<std::mutex> lock(g_wmu);
    auto it = g_wcache.find(k);
    if (it != g_wcache.end()) return pin(k, it->second).raw;
    const int fmt = src_fmt == eif::kSrcInt4 ? eif::kF32Int4 : (src_fmt == eif::kSrcInt8 ? eif::kF32Int8 : eif::kF32Tern);
    WEntry e;
    e.bytes = eif::f32_tiles_bytes(fmt, rows, cols);
    make_room(e.bytes + n);
    DevBuf tmp, raw;
    DIE_ON(hipMalloc(&tmp.p, n ? n : 16), fn);
    DIE_ON(hipMalloc(&raw.p, e.bytes), fn);
    DIE_ON(hipMemcpyAsync(tmp.p, host, n, hipMemcpyHostToDevice, c.st), fn);
    DIE_RC(eif::launch_f32_repack(src_fmt, (const uint8_t *)tmp.p, raw.p, rows, cols, c.st), fn);
    DIE_ON(hipStreamSynchronize(c.st), fn);
    DIE_ON(hipFree(tmp.release()), fn);
    e.raw = raw.release();
    return insert(k, e).raw;
}

// The [tile][block][4 rows] copy of block scales [rows, ceil(cols / block)] (f32linear.hip), kept like weights.
const void *resident_block_scales(const float *host, int rows, int cols, int block, const char *fn)
{
    ThreadCtx &c = ctx(fn);
    const size_t n = sizeof(float) * (size_t)rows * (size_t)((cols + block - 1) / block);
    WKey k{host, n, kBlockScales, rows, block};
    std::lock_guard<std::mutex> lock(g_wmu);
    auto it = g_wcache.find(k);
    if (it != g_wcache.end()) return pin(k, it->second).raw;
    WEntry e;
    e.bytes = eif::f32_scales_bytes(rows, cols, block);
    make_room(e.bytes + n);
    DevBuf tmp, raw;
    DIE_ON(hipMalloc(&tmp.p, n), fn);
    DIE_ON(hipMalloc(&raw.p, e.bytes), fn);
    DIE_ON(hipMemcpyAsync(tmp.p, host, n, hipMemcpyHostToDevice, c.st), fn);
    DIE_RC(eif::launch_f32_scales((const float *)tmp.p, raw.p, rows, cols, block, c.st), fn);
    DIE_ON(hipStreamSynchronize(c.st), fn);
    DIE_ON(hipFree(tmp.release()), fn);
    e.raw = raw.release();
    return insert(k, e).raw;
}

const eif_hip_qweight *resident_tern_row(const uint8_t *host, int rows, int cols, const char *fn)
{
    ThreadCtx &c = ctx(fn);
    const size_t n = (size_t)rows * ((cols + 3) / 4);
    WKey k{host, n, kQTernRow, rows, cols};
    std::lock_guard<std::mutex> lock(g_wmu);
    auto it = g_wcache.find(k);
    if (it != g_wcache.end()) return pin(k, it->second).q;
    WEntry e;
    make_room(n + n / 8);   // the GPU layout is about the reference's size
    eif_hip_qweight *q = nullptr;
    DIE_RC(eif_hip_qweight_create(&q, EIF_HIP_W_TERNARY, rows, cols, 0, host, nullptr, 0, c.st), fn);
    std::unique_ptr<eif_hip_qweight, void (*)(eif_hip_qweight *)> own(q, eif_hip_qweight_destroy);
    size_t qb = 0;
    eif_hip_qweight_info(q, nullptr, nullptr, nullptr, nullptr, &qb);
    e.bytes = qb;
    e.q = q;
    WEntry &ins = insert(k, e);
    own.release();
    return ins.q;
}

float norm_fastmath(int block)
{
#if defined(__x86_64__)
    // gcc -O3 -mavx2 -mfma -ffast-math evaluates 1.0f/sqrtf(a) as rsqrtss then fma(a*x0, x0, -3) * (x0 * -0.5).
    const float a = (float)block;
    const float x0 = _mm_cvtss_f32(_mm_rsqrt_ss(_mm_set_ss(a)));
    const float e0 = a * x0;
    const float e1 = fmaf(e0, x0, -3.0f);
    const float e2 = x0 * -0.5f;
    return e1 * e2;
#else
    return (float)(1.0 / sqrt((double)block));
#endif
}

bool pow2(int b) { return b > 0 && (b & (b - 1)) == 0; }

}  // namespace

extern "C" {

// ---- device layer helpers (eif_hip.h) ----

int eif_hip_init(int device)
{
    DevState &d = dev_state();
    if (!d.ok) return EIF_HIP_E_DEVICE;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return EIF_HIP_E_ARG;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) != hipSuccess || strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return EIF_HIP_E_DEVICE;
    if (hipSetDevice(device) != hipSuccess) return EIF_HIP_E_DEVICE;
    return eif::scratch_init(device, nullptr);   // the no-alloc entry point's scratch address on this device
}

const char *eif_hip_strerror(int code)
{
    switch (code) {
    case EIF_HIP_OK: return "ok";
    case EIF_HIP_E_ARG: return "invalid argument";
    case EIF_HIP_E_DEVICE: return "HIP device or runtime error";
    case EIF_HIP_E_NOMEM: return "device allocation failed";
    case EIF_HIP_E_LIMIT: return "request beyond a documented limit";
    default: return "unknown error";
    }
}

float eif_hip_wht_norm(int block) { return block > 0 ? norm_fastmath(block) : 1.0f; }

float eif_hip_wht_norm_exact(int block) { return block > 0 ? (float)(1.0 / sqrt((double)block)) : 1.0f; }

size_t eif_hip_set_host_weight_cache_limit(size_t bytes)
{
    std::lock_guard<std::mutex> lock(g_wmu);
    const size_t old = g_cache_limit;
    g_cache_limit = bytes;
    return old;
}

size_t eif_hip_host_weight_cache_bytes(void)
{
    std::lock_guard<std::mutex> lock(g_wmu);
    return g_cache_bytes;
}

int eif_hip_set_host_error_mode(int mode)
{
    if (mode != EIF_HIP_HOST_ABORT && mode != EIF_HIP_HOST_RECORD) return -1;
    return g_host_err_mode.exchange(mode);
}

int eif_hip_host_last_error(char *msg, size_t len)
{
    const int code = t_err_code;
    if (msg && len) snprintf(msg, len, "%s", code == EIF_HIP_OK ? "" : t_err_msg);
    t_err_code = EIF_HIP_OK;
    return code;
}

void eif_hip_forget_host_weights(const void *host_ptr)
{
    std::lock_guard<std::mutex> lock(g_wmu);
    for (auto it = g_wcache.begin(); it != g_wcache.end();) {
        if (host_ptr == nullptr || it->first.p == host_ptr) {
            g_cache_bytes -= it->second.bytes;
            free_entry(it->second);
            it = g_wcache.erase(it);
        } else {
            ++it;
        }
    }
}

// ---- format and size helpers (byte packing on the host; no arithmetic kernel involved) ----
// src/eif_quantize_bitnet.c:15-41, :92-112, :1422-1456, :1527-1541

int8_t eif_unpack_ternary(uint8_t byte, int pos)
{
    const unsigned code = (byte >> (2 * pos)) & 3u;
    return code == 1u ? 1 : (code == 2u ? -1 : 0);
}

size_t eif_pack_ternary(const int8_t *ternary, uint8_t *packed, size_t count)
{
    const size_t nb = (count + 3) / 4;
    for (size_t b = 0; b < nb; ++b) {
        unsigned v = 0;
        for (unsigned p = 0; p < 4; ++p) {
            const size_t i = 4 * b + p;
            if (i < count && ternary[i]) v |= (ternary[i] > 0 ? 1u : 2u) << (2 * p);
        }
        packed[b] = (uint8_t)v;
    }
    return nb;
}

size_t eif_pack_ternary_dense(const int8_t *ternary, uint8_t *packed, size_t count)
{
    const size_t nb = (count + 4) / 5;
    for (size_t b = 0; b < nb; ++b) {
        unsigned v = 0, mul = 1;
        for (unsigned p = 0; p < 5; ++p, mul *= 3) {
            const size_t i = 5 * b + p;
            if (i < count && ternary[i]) v += (ternary[i] > 0 ? 1u : 2u) * mul;
        }
        packed[b] = (uint8_t)v;
    }
    return nb;
}

size_t eif_interleave_weights_4rows(const uint8_t *src, uint8_t *dst, int rows, int cols)
{
    if (!src || !dst || rows <= 0 || cols <= 0) return 0;
    const size_t ng = (size_t)(cols + 3) / 4;
    size_t off = 0;
    int r = 0;
    for (; r < (rows & ~3); r += 4)
        for (size_t g = 0; g < ng; ++g)
            for (int k = 0; k < 4; ++k) dst[off++] = src[(size_t)(r + k) * ng + g];
    for (; r < rows; ++r, off += ng) memcpy(dst + off, src + (size_t)r * ng, ng);
    return off;
}

int eif_hadamard_block_size(int n)
{
    int b = 1;
    while (n > 0 && n % (2 * b) == 0 && 2 * b <= 1024) b *= 2;
    return b;
}

int eif_bitnet_group_size(int n, int max_group)
{
    if (max_group <= 0 || max_group >= n) return 0;
    for (int g = max_group - max_group % 32; g >= 32; g -= 32)
        if (n % g == 0) return g;
    return 0;
}

// ---- activation prep ----

void eif_hadamard_rotate_f32(float *x, const float *signs, int n, int block) try
{
    static const char *fn = "eif_hadamard_rotate_f32";
    if (!x || block <= 0 || n % block != 0 || !pow2(block)) return;
    ThreadCtx &c = call_ctx(fn);
    float *dx = (float *)upload(c, 0, x, sizeof(float) * n, fn);
    const float *ds = (const float *)upload(c, 1, signs, sizeof(float) * n, fn);
    DIE_RC(eif::launch_rotate_rows(dx, n, ds, 1, n, block, eif_hip_wht_norm(block), c.st), fn);
    download_sync(c, x, dx, sizeof(float) * n, fn);
} catch (const HostError &) {}

void eif_quantize_activation_i8(const float *x_f32, int8_t *x_i8, float *out_scale, int n) try
{
    static const char *fn = "eif_quantize_activation_i8";
    if (n <= 0) {
        if (out_scale) *out_scale = 1.0f;
        return;
    }
    ThreadCtx &c = call_ctx(fn);
    const float *dx = (const float *)upload(c, 0, x_f32, sizeof(float) * n, fn);
    int8_t *dq = (int8_t *)slot(c, 1, (size_t)n, fn);
    float *ds = (float *)slot(c, 2, sizeof(float), fn);
    DIE_RC(eif::launch_quant_rows(dx, n, 1, n, dq, n, ds, c.st), fn);
    float s = 1.0f;
    DIE_ON(hipMemcpyAsync(&s, ds, sizeof(float), hipMemcpyDeviceToHost, c.st), fn);
    download_sync(c, x_i8, dq, (size_t)n, fn);
    if (out_scale) *out_scale = s;
} catch (const HostError &) {}

// ---- INT8-activation ternary (MFMA kernel, resident repacked codes) ----

static void i8xternary(const char *fn, const uint8_t *w, const float *scales, const int8_t *xq_host,
                       const float *x_host, float scale_in, const float *bias, float *out, int rows, int cols)
{
    PinScope pins;
    ThreadCtx &c = call_ctx(fn);
    const eif_hip_qweight *q = resident_tern_row(w, rows, cols, fn);
    int kpad = 0;
    eif_hip_qweight_info(q, nullptr, nullptr, &kpad, nullptr, nullptr);
    int8_t *dq = (int8_t *)slot(c, 0, (size_t)kpad, fn);
    float *dxs = (float *)slot(c, 1, sizeof(float), fn);
    if (xq_host) {
        DIE_ON(hipMemsetAsync(dq, 0, (size_t)kpad, c.st), fn);
        DIE_ON(hipMemcpyAsync(dq, xq_host, (size_t)cols, hipMemcpyHostToDevice, c.st), fn);
        DIE_ON(hipMemcpyAsync(dxs, &scale_in, sizeof(float), hipMemcpyHostToDevice, c.st), fn);
    } else {
        const float *dx = (const float *)upload(c, 2, x_host, sizeof(float) * cols, fn);
        DIE_RC(eif::launch_prep_rows(dx, cols, nullptr, 1, cols, 0, 1.0f, dq, kpad, dxs, nullptr, 0, c.st), fn);
    }
    const float *dsc = (const float *)upload(c, 3, scales, sizeof(float) * rows, fn);
    const float *db = (const float *)upload(c, 4, bias, sizeof(float) * rows, fn);
    float *dy = (float *)out_slot(c, 5, sizeof(float) * rows, fn);
    DIE_RC(eif::qlinear_scaled(q, dsc, dq, kpad, dxs, db, dy, rows, 1, EIF_HIP_PATH_GEMV, c.st), fn);
    download_sync(c, out, dy, sizeof(float) * rows, fn);
    if (xq_host) DIE_ON(hipStreamSynchronize(c.st), fn);
}

void eif_matmul_bitnet_i8xternary_f32(const uint8_t *weights, const float *scales, const int8_t *input_i8,
                                      float scale_in, const float *bias, float *output, int rows, int cols) try
{
    if (!weights || !input_i8 || !output || rows <= 0 || cols <= 0) return;
    i8xternary("eif_matmul_bitnet_i8xternary_f32", weights, scales, input_i8, nullptr, scale_in, bias, output,
               rows, cols);
} catch (const HostError &) {}

void eif_matmul_bitnet_act_quant_f32(const uint8_t *weights, const float *scales, const float *input_f32,
                                     const float *bias, float *output, int rows, int cols) try
{
    if (!weights || !input_f32 || !output || rows <= 0 || cols <= 0) return;
    i8xternary("eif_matmul_bitnet_act_quant_f32", weights, scales, nullptr, input_f32, 1.0f, bias, output, rows,
               cols);
} catch (const HostError &) {}

void eif_matmul_bitnet_int8(const uint8_t *weights, float scale_w, const int8_t *input, float scale_in,
                            const int32_t *bias, int8_t *output, float scale_out, int rows, int cols) try
{
    static const char *fn = "eif_matmul_bitnet_int8";
    PinScope pins;
    if (!weights || !input || !output || rows <= 0 || cols <= 0) return;
    ThreadCtx &c = call_ctx(fn);
    const float eff = (scale_w * scale_in) / (scale_out > 1e-12f ? scale_out : 1.0f);
    const uint8_t *dw = (const uint8_t *)resident_raw(weights, (size_t)rows * ((cols + 3) / 4), fn);
    const int8_t *dx = (const int8_t *)upload(c, 0, input, (size_t)cols, fn);
    const int32_t *db = (const int32_t *)upload(c, 1, bias, sizeof(int32_t) * rows, fn);
    int8_t *dy = (int8_t *)out_slot(c, 2, (size_t)rows, fn);
    DIE_RC(eif::launch_tern_int8_out(dw, dx, db, dy, eff, rows, cols, c.st), fn);
    download_sync(c, output, dy, (size_t)rows, fn);
} catch (const HostError &) {}

// ---- FP32-activation ternary (the reference engines' x86 path) ----

static void tern_f32(const char *fn, const uint8_t *w, size_t wbytes, const float *scales, size_t nsc, int mode,
                     int block, const float *x, const float *bias, float *out, int rows, int cols, int il)
{
    PinScope pins;
    ThreadCtx &c = call_ctx(fn);
    const bool tiles = eif::f32_tiles_fit(cols, mode ? block : 0);
    const void *dw = tiles ? resident_tiles(w, wbytes, il ? eif::kSrcTernIl : eif::kSrcTernRow, rows, cols, fn)
                           : resident_raw(w, wbytes, fn);
    const float *dx = (const float *)upload(c, 0, x, sizeof(float) * cols, fn);
    const float *dsc = tiles && mode && scales ? (const float *)resident_block_scales(scales, rows, cols, block, fn)
                                               : (const float *)upload(c, 1, scales, sizeof(float) * nsc, fn);
    const float *db = (const float *)upload(c, 2, bias, sizeof(float) * rows, fn);
    float *dy = (float *)out_slot(c, 3, sizeof(float) * rows, fn);
    if (tiles)
        DIE_RC(eif::launch_f32_tiles(eif::kF32Tern, dw, dsc, mode ? block : 0, dx, db, dy, rows, cols, c.st), fn);
    else
        DIE_RC(eif::launch_tern_f32((const uint8_t *)dw, dsc, mode, block, dx, db, dy, rows, cols, il, c.st), fn);
    download_sync(c, out, dy, sizeof(float) * rows, fn);
}

void eif_matmul_bitnet_f32(const uint8_t *weights, const float *scales, const float *input, const float *bias,
                           float *output, int rows, int cols) try
{
    if (!weights || !input || !output || rows <= 0 || cols <= 0) return;
    tern_f32("eif_matmul_bitnet_f32", weights, (size_t)rows * ((cols + 3) / 4), scales, (size_t)rows, 0, 0, input,
             bias, output, rows, cols, 0);
} catch (const HostError &) {}

bool eif_gpu_matmul_bitnet_f32(eif_gpu_context_t *ctx, const uint8_t *weights, const float *scales,
                               const float *input, const float *bias, float *output, int rows, int cols) try
{
    (void)ctx;
    if (!weights || !input || !output || rows <= 0 || cols <= 0 || !dev_state().ok) return false;
    ForceRecord rec;   // a failure returns false (the caller runs its CPU kernel), never aborts
    tern_f32("eif_gpu_matmul_bitnet_f32", weights, (size_t)rows * ((cols + 3) / 4), scales, (size_t)rows, 0, 0,
             input, bias, output, rows, cols, 0);
    return true;
} catch (const HostError &) {
    return false;
}

void eif_matmul_bitnet_block_f32(const uint8_t *weights, const float *block_scales, int block_size,
                                 const float *input, const float *bias, float *output, int rows, int cols) try
{
    if (!weights || !input || !output || rows <= 0 || cols <= 0) return;
    if (block_size <= 0) block_size = 64;
    const size_t nb = (size_t)((cols + block_size - 1) / block_size);
    tern_f32("eif_matmul_bitnet_block_f32", weights, (size_t)rows * ((cols + 3) / 4), block_scales, rows * nb, 1,
             block_size, input, bias, output, rows, cols, 0);
} catch (const HostError &) {}

void eif_matmul_bitnet_f32_w1w3(float *out_w1, float *out_w3, const uint8_t *w1, const uint8_t *w3,
                                const float *scale_w1, const float *scale_w3, const float *input, int hidden_dim,
                                int dim) try
{
    if (!out_w1 || !out_w3 || !w1 || !w3 || !input || hidden_dim <= 0 || dim <= 0) return;
    const size_t wb = (size_t)hidden_dim * ((dim + 3) / 4);
    tern_f32("eif_matmul_bitnet_f32_w1w3", w1, wb, scale_w1, (size_t)hidden_dim, 0, 0, input, nullptr, out_w1,
             hidden_dim, dim, 0);
    tern_f32("eif_matmul_bitnet_f32_w1w3", w3, wb, scale_w3, (size_t)hidden_dim, 0, 0, input, nullptr, out_w3,
             hidden_dim, dim, 0);
} catch (const HostError &) {}

void eif_matmul_bitnet_tmac_interleaved_f32(const uint8_t *interleaved_weights, const float *scales,
                                           const float *input, const float *bias, float *output, int rows,
                                           int cols) try
{
    if (!interleaved_weights || !input || !output || rows <= 0 || cols <= 0) return;
    tern_f32("eif_matmul_bitnet_tmac_interleaved_f32", interleaved_weights, (size_t)rows * ((cols + 3) / 4), scales,
             (size_t)rows, 0, 0, input, bias, output, rows, cols, 1);
} catch (const HostError &) {}

void eif_matmul_bitnet_dense_f32(const uint8_t *weights, const float *scales, const float *input,
                                 const float *bias, float *output, int rows, int cols) try
{
    static const char *fn = "eif_matmul_bitnet_dense_f32";
    PinScope pins;
    if (!weights || !input || !output || rows <= 0 || cols <= 0) return;
    ThreadCtx &c = call_ctx(fn);
    const size_t wb = (size_t)rows * ((cols + 4) / 5);
    const bool tiles = eif::f32_tiles_fit(cols, 0);
    const void *dw = tiles ? resident_tiles(weights, wb, eif::kSrcDense, rows, cols, fn) : resident_raw(weights, wb, fn);
    const float *dx = (const float *)upload(c, 0, input, sizeof(float) * cols, fn);
    const float *dsc = (const float *)upload(c, 1, scales, sizeof(float) * rows, fn);
    const float *db = (const float *)upload(c, 2, bias, sizeof(float) * rows, fn);
    float *dy = (float *)out_slot(c, 3, sizeof(float) * rows, fn);
    if (tiles)
        DIE_RC(eif::launch_f32_tiles(eif::kF32Tern, dw, dsc, 0, dx, db, dy, rows, cols, c.st), fn);
    else
        DIE_RC(eif::launch_dense_f32((const uint8_t *)dw, dsc, dx, db, dy, rows, cols, c.st), fn);
    download_sync(c, output, dy, sizeof(float) * rows, fn);
} catch (const HostError &) {}

// ---- INT8 / INT4 row-scaled, FP32 activations ----

static void int_f32(const char *fn, bool int4, const void *w, const float *sc, const float *x, float *out, int rows,
                    int cols)
{
    PinScope pins;
    ThreadCtx &c = call_ctx(fn);
    const size_t wb = int4 ? (size_t)rows * ((cols + 1) / 2) : (size_t)rows * cols;
    const bool tiles = eif::f32_tiles_fit(cols, 0);
    const void *dw = tiles ? resident_tiles(w, wb, int4 ? eif::kSrcInt4 : eif::kSrcInt8, rows, cols, fn)
                           : resident_raw(w, wb, fn);
    const float *dx = (const float *)upload(c, 0, x, sizeof(float) * cols, fn);
    const float *dsc = (const float *)upload(c, 1, sc, sizeof(float) * rows, fn);
    float *dy = (float *)out_slot(c, 2, sizeof(float) * rows, fn);
    if (tiles)
        DIE_RC(eif::launch_f32_tiles(int4 ? eif::kF32Int4 : eif::kF32Int8, dw, dsc, 0, dx, nullptr, dy, rows, cols, c.st),
               fn);
    else if (int4)
        DIE_RC(eif::launch_int4_f32((const uint8_t *)dw, dsc, dx, dy, rows, cols, c.st), fn);
    else
        DIE_RC(eif::launch_int8_f32((const int8_t *)dw, dsc, dx, dy, rows, cols, c.st), fn);
    download_sync(c, out, dy, sizeof(float) * rows, fn);
}

void tinyllm_matmul_int8_rowscale(float *y, const int8_t *w, const float *x, int in_dim, int out_dim,
                                  const float *scales) try
{
    if (!y || !w || !x || in_dim <= 0 || out_dim <= 0) return;
    int_f32("tinyllm_matmul_int8_rowscale", false, w, scales, x, y, out_dim, in_dim);
} catch (const HostError &) {}

void eif_int8_gemv_f32(float *out, const int8_t *W, const float *sc, const float *x, int rows, int cols) try
{
    if (!out || !W || !x || rows <= 0 || cols <= 0) return;
    int_f32("eif_int8_gemv_f32", false, W, sc, x, out, rows, cols);
} catch (const HostError &) {}

void eif_int4_gemv_f32(float *out, const uint8_t *W, const float *sc, const float *x, int rows, int cols) try
{
    if (!out || !W || !x || rows <= 0 || cols <= 0) return;
    int_f32("eif_int4_gemv_f32", true, W, sc, x, out, rows, cols);
} catch (const HostError &) {}

// ---- FP32 GEMM and softmax ----

void eif_gemm_f32_nt_ld(const float *A, int lda, const float *W, int ldw, const float *bias, float *C, int ldc,
                        int M, int N, int K, int act, int accumulate) try
{
    static const char *fn = "eif_gemm_f32_nt_ld";
    if (M <= 0 || N <= 0 || !C) return;
    if (K > 0 && (!A || !W)) return;
    ThreadCtx &c = call_ctx(fn);
    float *dA = nullptr, *dW = nullptr;
    if (K > 0) {
        dA = (float *)slot(c, 0, sizeof(float) * (size_t)M * K, fn);
        dW = (float *)slot(c, 1, sizeof(float) * (size_t)N * K, fn);
        DIE_ON(hipMemcpy2DAsync(dA, sizeof(float) * K, A, sizeof(float) * lda, sizeof(float) * K, M,
                                hipMemcpyHostToDevice, c.st), fn);
        DIE_ON(hipMemcpy2DAsync(dW, sizeof(float) * K, W, sizeof(float) * ldw, sizeof(float) * K, N,
                                hipMemcpyHostToDevice, c.st), fn);
    }
    const float *db = (const float *)upload(c, 2, bias, sizeof(float) * N, fn);
    float *dC = (float *)slot(c, 3, sizeof(float) * (size_t)M * N, fn);
    if (accumulate)
        DIE_ON(hipMemcpy2DAsync(dC, sizeof(float) * N, C, sizeof(float) * ldc, sizeof(float) * N, M,
                                hipMemcpyHostToDevice, c.st), fn);
    DIE_RC(eif::launch_gemm_f32_nt(dA, K, dW, K, db, dC, N, M, N, K > 0 ? K : 0, act, accumulate, c.st), fn);
    DIE_ON(hipMemcpy2DAsync(C, sizeof(float) * ldc, dC, sizeof(float) * N, sizeof(float) * N, M,
                            hipMemcpyDeviceToHost, c.st), fn);
    DIE_ON(hipStreamSynchronize(c.st), fn);
} catch (const HostError &) {}

void eif_gemm_f32_nt(const float *A, const float *W, const float *bias, float *C, int M, int N, int K, int act,
                     int accumulate)
{
    eif_gemm_f32_nt_ld(A, K, W, K, bias, C, N, M, N, K, act, accumulate);
}

void eif_softmax_rows_f32(float *S, int rows, int cols, int ld, float scale) try
{
    static const char *fn = "eif_softmax_rows_f32";
    if (!S || rows <= 0 || cols <= 0 || ld < cols) return;
    ThreadCtx &c = call_ctx(fn);
    float *dS = (float *)slot(c, 0, sizeof(float) * (size_t)rows * cols, fn);
    DIE_ON(hipMemcpy2DAsync(dS, sizeof(float) * cols, S, sizeof(float) * ld, sizeof(float) * cols, rows,
                            hipMemcpyHostToDevice, c.st), fn);
    DIE_RC(eif::launch_softmax_rows(dS, rows, cols, cols, scale, c.st), fn);
    DIE_ON(hipMemcpy2DAsync(S, sizeof(float) * ld, dS, sizeof(float) * cols, sizeof(float) * cols, rows,
                            hipMemcpyDeviceToHost, c.st), fn);
    DIE_ON(hipStreamSynchronize(c.st), fn);
} catch (const HostError &) {}

}  // extern "C"
