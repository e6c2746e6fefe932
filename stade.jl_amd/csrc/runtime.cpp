// libstade_hip runtime: last-error state, per-device workspace, library info, stack
// allocation helpers and the input generator (Julia's Xoshiro stream, host side).
#include "internal.hpp"
#include "../../include/stade_hip.h"

#include <map>
#include <mutex>
#include <string>
#include <vector>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <math.h>

namespace stade {

static thread_local char g_err[512] = "";

int32_t set_error(int32_t code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int32_t check_hip(hipError_t e, const char* what) {
    return set_error((int32_t)e, "%s: %s (hipError %d)", what, hipGetErrorString(e), (int)e);
}

static std::mutex g_ws_mu;
static Workspace g_ws[64];
static bool g_ws_ready[64];

// per device: the lock a library call holds while it enqueues, and the event the last call
// recorded on its stream at its end
static std::recursive_mutex g_call_mu[64];
struct CallOrder {
    hipStream_t last;
    bool has_last;
    hipEvent_t ev;
};
static CallOrder g_order[64];
// whether the library call running on this thread enqueues under graph capture
static thread_local bool tl_capturing = false;
static thread_local int32_t tl_scratch_code = STADE_HIP_ENOMEM;
// scratch buffers replaced while a captured graph may still hold their addresses: kept for
// the life of the process (each retirement follows a growth, so they total less than the
// largest scratch ever requested times two)
static std::vector<void*> g_retired;

Workspace* workspace() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        check_hip(e, "hipGetDevice");
        return nullptr;
    }
    if (dev < 0 || dev >= 64) {
        set_error(STADE_HIP_ERANGE, "device ordinal %d out of range", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if (!g_ws_ready[dev]) {
        Workspace w{};
        if ((e = hipMalloc(&w.partials, sizeof(double) * kPartialSlots)) != hipSuccess ||
            (e = hipMalloc(&w.dscalars, sizeof(double) * kDeviceScalars)) != hipSuccess ||
            (e = hipMemset(w.dscalars, 0, sizeof(double) * kDeviceScalars)) != hipSuccess ||
            (e = hipMalloc(&w.sync, sizeof(uint32_t) * kSyncSlots)) != hipSuccess ||
            (e = hipMemset(w.sync, 0, sizeof(uint32_t) * kSyncSlots)) != hipSuccess ||
            (e = hipDeviceSynchronize()) != hipSuccess) {
            check_hip(e, "workspace allocation");
            return nullptr;
        }
        g_ws[dev] = w;
        g_ws_ready[dev] = true;
    }
    return &g_ws[dev];
}

WsCall::WsCall(hipStream_t stream, bool with_workspace)
    : ws(nullptr), dev_(-1), stream_(stream), capturing_(false), ok_(false), err_(STADE_HIP_ENOMEM) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        err_ = check_hip(e, "hipGetDevice");
        return;
    }
    if (dev < 0 || dev >= 64) {
        err_ = set_error(STADE_HIP_ERANGE, "device ordinal %d out of range", dev);
        return;
    }
    g_call_mu[dev].lock();
    dev_ = dev;
    Workspace* w = with_workspace ? workspace() : nullptr;
    if (with_workspace && !w) {
        err_ = STADE_HIP_ENOMEM;
        return;
    }
    CallOrder& o = g_order[dev];
    // a stream under graph capture takes no dependency on work outside the capture: such
    // calls are ordered by the graph the caller builds
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    capturing_ = hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    tl_capturing = capturing_;
    if (capturing_ && w) w->scratch_captured = true;
    if (!capturing_ && o.has_last && o.last != stream && o.ev) {
        if ((e = hipStreamWaitEvent(stream, o.ev, 0)) != hipSuccess) {
            err_ = check_hip(e, "hipStreamWaitEvent (ordering after the previous call's stream)");
            return;
        }
    }
    ws = w;
    ok_ = true;
}

int32_t call_order_setup() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return check_hip(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return set_error(STADE_HIP_ERANGE, "device ordinal %d out of range", dev);
    std::lock_guard<std::recursive_mutex> lk(g_call_mu[dev]);
    CallOrder& o = g_order[dev];
    if (!o.ev && (e = hipEventCreateWithFlags(&o.ev, hipEventDisableTiming)) != hipSuccess)
        return check_hip(e, "hipEventCreateWithFlags (call order)");
    return 0;
}

WsCall::~WsCall() {
    if (dev_ < 0) return;
    tl_capturing = false;
    if (ok_ && !capturing_) {
        CallOrder& o = g_order[dev_];
        hipError_t e = hipSuccess;
        if (!o.ev) e = hipEventCreateWithFlags(&o.ev, hipEventDisableTiming);
        // a failure leaves the next call on another stream unordered; it is reported by
        // that call's own first HIP error, if any
        if (e == hipSuccess) (void)hipEventRecord(o.ev, stream_);
        o.last = stream_;
        o.has_last = true;
    }
    g_call_mu[dev_].unlock();
}

void* scratch(size_t bytes) {
    Workspace* w = workspace();
    if (!w) return nullptr;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if (w->scratch_bytes < bytes) {
        if (tl_capturing) {
            tl_scratch_code = STADE_HIP_ESTATE;
            set_error(STADE_HIP_ESTATE,
                      "the library workspace cannot grow under graph capture (%zu bytes needed, %zu held): "
                      "make one eager call of the largest size before capturing", bytes, w->scratch_bytes);
            return nullptr;
        }
        if (w->scratch) {
            if (w->scratch_captured) {
                // a captured graph may replay with this address: keep the buffer
                g_retired.push_back(w->scratch);
            } else {
                // wait for kernels still using the old buffer; a failure here is sticky and is
                // reported by the next launch's status
                (void)hipDeviceSynchronize();
                (void)hipFree(w->scratch);
            }
            w->scratch = nullptr;
            w->scratch_bytes = 0;
        }
        hipError_t e = hipMalloc(&w->scratch, bytes);
        if (e != hipSuccess) {
            tl_scratch_code = STADE_HIP_ENOMEM;
            check_hip(e, "scratch allocation");
            return nullptr;
        }
        w->scratch_bytes = bytes;
        w->scratch_captured = false;
    }
    return w->scratch;
}

int32_t scratch_error() { return tl_scratch_code; }

// ------------------------------------------------------------------------------------------
// kernel timing
// ------------------------------------------------------------------------------------------
struct ProfPending {
    std::string name;
    hipEvent_t a, b;
};
static std::mutex g_prof_mu;
static bool g_prof_on = false;
static std::vector<hipEvent_t> g_ev_pool;
static std::vector<ProfPending> g_pending;
static std::map<std::string, std::pair<double, int64_t>> g_prof_tot;
static thread_local ProfPending g_open;

static hipEvent_t ev_get() {
    if (!g_ev_pool.empty()) {
        hipEvent_t e = g_ev_pool.back();
        g_ev_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    (void)hipEventCreate(&e);  // profiling only: a failed event records nothing
    return e;
}

bool prof_enabled() { return g_prof_on; }

void prof_begin(const char* kernel, hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_open.name = kernel;
    g_open.a = ev_get();
    g_open.b = ev_get();
    (void)hipEventRecord(g_open.a, s);
}

void prof_end(hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    (void)hipEventRecord(g_open.b, s);
    g_pending.push_back(g_open);
}

static void prof_collect_locked() {
    for (auto& p : g_pending) {
        float ms = 0.f;
        if (hipEventSynchronize(p.b) == hipSuccess && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            auto& t = g_prof_tot[p.name];
            t.first += ms;
            t.second += 1;
        }
        g_ev_pool.push_back(p.a);
        g_ev_pool.push_back(p.b);
    }
    g_pending.clear();
}

// ------------------------------------------------------------------------------------------
// Julia's Random.Xoshiro scalar stream (Julia 1.10): seeding by SHA-256 of the seed's 32-bit
// little-endian words, xoshiro256++ steps, Float64 = (next >>> 11) * 2^-53.  The normal draw
// is STADE's `val_normal` (/root/reference/src/STADE.jl:16628-16637): Box-Muller, cosine
// branch, u1 = 1 - rand(), u2 = rand().
// ------------------------------------------------------------------------------------------
namespace sha {
static const uint32_t K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
static inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
// SHA-256 of a short message (at most 55 bytes: one block).
static void digest(const uint8_t* msg, size_t len, uint8_t out[32]) {
    uint8_t blk[64] = {0};
    memcpy(blk, msg, len);
    blk[len] = 0x80;
    uint64_t bits = (uint64_t)len * 8;
    for (int i = 0; i < 8; ++i) blk[63 - i] = (uint8_t)(bits >> (8 * i));
    uint32_t w[64];
    for (int i = 0; i < 16; ++i)
        w[i] = (uint32_t)blk[4 * i] << 24 | (uint32_t)blk[4 * i + 1] << 16 | (uint32_t)blk[4 * i + 2] << 8 | blk[4 * i + 3];
    for (int i = 16; i < 64; ++i) {
        uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; ++i) {
        uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
        uint32_t ch = (e & f) ^ (~e & g);
        uint32_t t1 = hh + S1 + ch + K[i] + w[i];
        uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
        uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
        uint32_t t2 = S0 + mj;
        hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    for (int i = 0; i < 8; ++i) {
        out[4 * i] = (uint8_t)(h[i] >> 24);
        out[4 * i + 1] = (uint8_t)(h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(h[i] >> 8);
        out[4 * i + 3] = (uint8_t)h[i];
    }
}
}  // namespace sha

}  // namespace stade

using namespace stade;

extern "C" {

const char* stade_hip_last_error(void) { return g_err; }

const char* stade_hip_version(void) { return "stade_hip 0.1 (gfx950)"; }

uint64_t stade_hip_stable_seed(const char* name) {
    uint64_t h = 0xcbf29ce484222325ULL;
    for (const unsigned char* p = (const unsigned char*)name; *p; ++p) h = (h ^ *p) * 0x00000100000001b3ULL;
    return h;
}

int32_t stade_hip_rng_seed(uint64_t seed, uint64_t state[4]) {
    if (!state) return set_error(STADE_HIP_EINVAL, "stade_hip_rng_seed: null state");
    uint8_t msg[8];
    size_t len = 0;
    // the seed's 32-bit words, least significant first, at least one word
    do {
        uint32_t wd = (uint32_t)(seed & 0xffffffffu);
        memcpy(msg + len, &wd, 4);  // little-endian host
        len += 4;
        seed >>= 32;
    } while (seed != 0);
    uint8_t dg[32];
    sha::digest(msg, len, dg);
    memcpy(state, dg, 32);
    return STADE_HIP_OK;
}

static inline uint64_t xo_next(uint64_t s[4]) {
    uint64_t s0 = s[0], s1 = s[1], s2 = s[2], s3 = s[3];
    uint64_t tmp = s0 + s3;
    uint64_t res = ((tmp << 23) | (tmp >> 41)) + s0;
    uint64_t t = s1 << 17;
    s2 ^= s0;
    s3 ^= s1;
    s1 ^= s2;
    s0 ^= s3;
    s2 ^= t;
    s3 = (s3 << 45) | (s3 >> 19);
    s[0] = s0; s[1] = s1; s[2] = s2; s[3] = s3;
    return res;
}
static inline double xo_rand(uint64_t s[4]) { return (double)(xo_next(s) >> 11) * 0x1.0p-53; }

int32_t stade_hip_rng_normal_f64(uint64_t state[4], double* out, int64_t n) {
    if (!state || (!out && n > 0) || n < 0) return set_error(STADE_HIP_EINVAL, "stade_hip_rng_normal_f64: bad arguments");
    for (int64_t i = 0; i < n; ++i) {
        double u1 = 1.0 - xo_rand(state);
        double u2 = xo_rand(state);
        out[i] = sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2);
    }
    return STADE_HIP_OK;
}

int32_t stade_hip_rng_uniform_f64(uint64_t state[4], double* out, int64_t n, double lo, double hi) {
    if (!state || (!out && n > 0) || n < 0) return set_error(STADE_HIP_EINVAL, "stade_hip_rng_uniform_f64: bad arguments");
    for (int64_t i = 0; i < n; ++i) out[i] = lo + (hi - lo) * xo_rand(state);
    return STADE_HIP_OK;
}

int32_t stade_hip_rng_int_range(uint64_t state[4], int64_t* out, int64_t n, int64_t lo, int64_t hi) {
    // lo + floor(rand() * (hi - lo + 1)): the build's own documented integer draw
    if (!state || (!out && n > 0) || n < 0 || hi < lo) return set_error(STADE_HIP_EINVAL, "stade_hip_rng_int_range: bad arguments");
    const double span = (double)(hi - lo + 1);
    for (int64_t i = 0; i < n; ++i) {
        int64_t v = lo + (int64_t)floor(xo_rand(state) * span);
        out[i] = v > hi ? hi : v;
    }
    return STADE_HIP_OK;
}

int32_t stade_hip_profile_start(void) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    prof_collect_locked();
    g_prof_tot.clear();
    g_prof_on = true;
    return STADE_HIP_OK;
}

int32_t stade_hip_profile_stop(void) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof_on = false;
    return STADE_HIP_OK;
}

int32_t stade_hip_profile_read(const char* kernel, double* total_ms, int64_t* launches) {
    if (!kernel || !total_ms || !launches) return set_error(STADE_HIP_EINVAL, "stade_hip_profile_read: null argument");
    std::lock_guard<std::mutex> lk(g_prof_mu);
    prof_collect_locked();
    auto it = g_prof_tot.find(kernel);
    *total_ms = it == g_prof_tot.end() ? 0.0 : it->second.first;
    *launches = it == g_prof_tot.end() ? 0 : it->second.second;
    return STADE_HIP_OK;
}

int32_t stade_hip_device_error(int32_t* flag) {
    // the flag a kernel raises for an input the generated code would reject at run time (an
    // index out of range); reading it waits for the device and clears it
    if (!flag) return set_error(STADE_HIP_EINVAL, "stade_hip_device_error: null flag");
    Workspace* w = workspace();
    if (!w) return STADE_HIP_ENOMEM;
    // every stream's kernels first (the flag may be raised by a call on any stream)
    STADE_TRY_HIP(hipDeviceSynchronize());
    int32_t h = 0, z = 0;
    STADE_TRY_HIP(hipMemcpy(&h, (int32_t*)(w->dscalars + kErrFlagSlot), sizeof h, hipMemcpyDeviceToHost));
    STADE_TRY_HIP(hipMemcpy((int32_t*)(w->dscalars + kErrFlagSlot), &z, sizeof z, hipMemcpyHostToDevice));
    *flag = h;
    return STADE_HIP_OK;
}

int32_t stade_hip_workspace_info(int64_t* scratch_bytes, int64_t* retired) {
    if (!scratch_bytes || !retired) return set_error(STADE_HIP_EINVAL, "stade_hip_workspace_info: null output");
    Workspace* w = workspace();
    if (!w) return STADE_HIP_ENOMEM;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    *scratch_bytes = (int64_t)w->scratch_bytes;
    *retired = (int64_t)g_retired.size();
    return STADE_HIP_OK;
}

int32_t stade_hip_free(void* p) {
    if (!p) return STADE_HIP_OK;
    hipError_t e = hipFree(p);
    return e == hipSuccess ? STADE_HIP_OK : check_hip(e, "hipFree");
}

int32_t stade_hip_synchronize(hipStream_t stream) {
    hipError_t e = hipStreamSynchronize(stream);
    return e == hipSuccess ? STADE_HIP_OK : check_hip(e, "hipStreamSynchronize");
}

}  // extern "C"
