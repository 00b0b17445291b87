// Host side of the MI355X exact-integer linear backend: the C ABI declared in include/kt_hip.h.
//
// The backend layer is this build's counterpart of TcLinear<DeviceExec> (crates/02-runtime/kt-cuda/src/backend.rs:77-192
// with device.rs:119-197): it chooses the digit planes from the operand ranges, keeps packed weights resident by
// WeightId under an LRU byte budget, packs the activations on the device, runs the digit-plane MFMA product in
// k-chunks short enough that no int32 accumulator can wrap, and copies the i64 result back. One mutex per backend
// orders the calls and guards the scratch buffers and the cache (the reference's scratch and cache Mutexes).
//
// Compiled twice: libkt_hip.so (the product) and, with KT_HIP_PLANTS, libkt_hip_planted.so (the firing controls of
// backend.rs:31-40, for tests only).

#include <hip/hip_runtime.h>
#include <limits.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "kt_kernels.h"

namespace {

std::atomic<uint64_t> g_fallbacks{0};
std::atomic<uint64_t> g_next_id{1};

int64_t kp_of(int64_t k) { return (k + 63) / 64 * 64; }

// A device allocation that only grows (DevBuf::grow, kt-cuda/src/device.rs:101-106).
struct DevBuf {
    void* ptr = nullptr;
    size_t cap = 0;
    hipError_t grow(size_t bytes) {
        if (bytes <= cap) return hipSuccess;
        if (ptr) {
            hipError_t e = hipFree(ptr);
            ptr = nullptr;
            cap = 0;
            if (e != hipSuccess) return e;
        }
        hipError_t e = hipMalloc(&ptr, bytes);
        if (e != hipSuccess) {
            ptr = nullptr;
            return e;
        }
        cap = bytes;
        return hipSuccess;
    }
    void release() {
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        cap = 0;
    }
};

// The plane counts with a kernel instantiation: a code needing p balanced base-256 digits runs as 1, 3 or 5 planes.
int plane_class(int p) { return p <= 1 ? 1 : (p <= 3 ? 3 : 5); }

// The fewest balanced base-256 digits holding every code: 1 digit covers [-128, 127], each further digit maps a
// range [lo, hi] to [256 lo - 128, 256 hi + 127].
int digits_for(const int32_t* v, size_t n) {
    int32_t lo = 0, hi = 0;
    for (size_t i = 0; i < n; i++) {
        lo = v[i] < lo ? v[i] : lo;
        hi = v[i] > hi ? v[i] : hi;
    }
    int64_t mn = -128, mx = 127;
    for (int p = 1; p < 5; p++) {
        if (lo >= mn && hi <= mx) return p;
        mn = mn * 256 - 128;
        mx = mx * 256 + 127;
    }
    return 5;
}

// k-chunk of the int32 accumulators: a group sums at most min(px, pw) plane pairs per k, each at most 128^2 in
// magnitude, so floor((2^31 - 1) / (min(px,pw) * 16384)) terms cannot wrap; rounded down to 256.
int64_t flush_of(int px, int pw) {
    int64_t n = px < pw ? px : pw;
    return (2147483647LL / (n * 16384)) / 256 * 256;
}

struct Key {
    bool has_id;
    uint64_t id;
    size_t out, k;
    bool operator<(const Key& o) const {
        return std::tie(has_id, id, out, k) < std::tie(o.has_id, o.id, o.out, o.k);
    }
};

struct Entry {
    int8_t* planes;
    int pw;
    uint64_t bytes;
    uint64_t last_use;
};

const char* plant_name(int p) {
    switch (p) {
        case KT_PLANT_DROP_TOP: return "DropTopPlane";
        case KT_PLANT_WRONG_CARRY: return "WrongCarry";
        case KT_PLANT_NO_FLUSH: return "NoFlush";
        case KT_PLANT_CACHE_BY_SHAPE: return "CacheByShape";
        default: return "None";
    }
}

}  // namespace

struct kt_hip_backend {
    int dev = 0;
    std::string devname;
    uint64_t budget = 0;
    bool budget_given = false;
    int plant = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;
    std::map<Key, Entry> cache;
    uint64_t bytes = 0, tick = 0;
    DevBuf xcodes, xplanes, ydev, wcodes;
};

#define KT_TRY(expr)                          \
    do {                                      \
        hipError_t e_ = (expr);               \
        if (e_ != hipSuccess) return (int)e_; \
    } while (0)

extern "C" {

// ----------------------------------------------------------------------------------------------------------------
// Device layer (kt_cuda_* of crates/02-runtime/kt-cuda/src/digit_gemm.cu:86-147)
// ----------------------------------------------------------------------------------------------------------------

int kt_hip_device_count(int* n) {
    *n = 0;
    return (int)hipGetDeviceCount(n);
}

// The marketing name, or the gfx architecture where the runtime reports none (some hosts leave it empty).
static std::string device_name(const hipDeviceProp_t& p) {
    std::string n(p.name);
    if (n.empty()) n = std::string(p.gcnArchName).substr(0, std::string(p.gcnArchName).find(':'));
    return n.empty() ? std::string("device") : n;
}

int kt_hip_device_info(int dev, char* name, int len, int* major, int* minor, size_t* free_bytes) {
    hipDeviceProp_t p;
    KT_TRY(hipGetDeviceProperties(&p, dev));
    if (len > 0) {
        strncpy(name, device_name(p).c_str(), (size_t)len - 1);
        name[len - 1] = 0;
    }
    *major = p.major;
    *minor = p.minor;
    KT_TRY(hipSetDevice(dev));
    size_t total = 0;
    return (int)hipMemGetInfo(free_bytes, &total);
}

int kt_hip_alloc(int dev, size_t bytes, void** p) {
    KT_TRY(hipSetDevice(dev));
    return (int)hipMalloc(p, bytes);
}

int kt_hip_free(int dev, void* p) {
    KT_TRY(hipSetDevice(dev));
    return (int)hipFree(p);
}

int kt_hip_upload(int dev, void* dst, const void* src, size_t bytes) {
    KT_TRY(hipSetDevice(dev));
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
}

int kt_hip_download(int dev, void* dst, const void* src, size_t bytes) {
    KT_TRY(hipSetDevice(dev));
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
}

const char* kt_hip_error_string(int e) { return hipGetErrorString((hipError_t)e); }

int64_t kt_hip_kp(int64_t k) { return kp_of(k); }

int kt_hip_planes_for(const int32_t* codes, size_t n) { return plane_class(digits_for(codes, n)); }

int kt_hip_pack_planes(int dev, const int32_t* codes_dev, int64_t rows, int64_t k, int planes, int8_t* planes_dev,
                       void* stream) {
    if (planes != 1 && planes != 3 && planes != 5) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_pack_planes(codes_dev, rows, k, planes, 0, planes_dev, (hipStream_t)stream);
}

int64_t kt_hip_flush_k(int px, int pw) { return flush_of(px, pw); }

int kt_hip_digit_gemm(int dev, const int8_t* xa_dev, int px, const int8_t* wb_dev, int pw, int64_t* y_dev,
                      int64_t rows, int64_t out, int64_t k, int64_t flush_k, int drop_top, void* stream) {
    if (rows <= 0 || out <= 0) return 0;
    const int64_t kp = kp_of(k);
    if (rows > INT_MAX || out > INT_MAX || kp > INT_MAX) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    hipStream_t s = (hipStream_t)stream;
    if (k == 0) return (int)hipMemsetAsync(y_dev, 0, (size_t)rows * (size_t)out * 8, s);
    int64_t fk = flush_k <= 0 ? flush_of(px, pw) : flush_k;
    if (fk % 256) return (int)hipErrorInvalidValue;
    for (int64_t k0 = 0; k0 < kp; k0 += fk) {
        const int64_t k1 = kp - k0 < fk ? kp : k0 + fk;
        KT_TRY(kt::launch_plane_gemm(px, pw, xa_dev, wb_dev, y_dev, (int)rows, (int)out, (int)kp, (int)k0, (int)k1,
                                     k0 > 0, drop_top, s));
    }
    return 0;
}

// ----------------------------------------------------------------------------------------------------------------
// QuantLinear::forward_int on the device (layers.rs:275-328)
// ----------------------------------------------------------------------------------------------------------------

size_t kt_hip_quant_linear_workspace(int64_t rows, int64_t in_f, int64_t out_f, size_t off[KT_QL_WS_PARTS]) {
    size_t tmp[KT_QL_WS_PARTS];
    if (rows < 1 || in_f < 1 || out_f < 1) return 0;
    return kt::ql_workspace_bytes(rows, in_f, out_f, off ? off : tmp);
}

int kt_hip_quant_linear(int dev, const int32_t* x_dev, int64_t rows, int64_t in_f, const kt_hip_qscale* xs_dev,
                        const int8_t* w_planes_dev, int pw, int64_t out_f, int64_t w_mant, int32_t w_shift,
                        const int64_t* bias_dev, int64_t b_mant, int32_t b_shift, void* ws_dev, size_t ws_bytes,
                        int32_t* y_dev, kt_hip_qscale* os_dev, void* stream) {
    if (rows < 1 || in_f < 1 || out_f < 1 || (pw != 1 && pw != 3 && pw != 5) || w_mant < 0 || b_mant < 0)
        return (int)hipErrorInvalidValue;
    const int64_t kp = kp_of(in_f);
    if (rows * kp >= ((int64_t)1 << 31) || rows * out_f >= ((int64_t)1 << 31) || kp > INT_MAX)
        return (int)hipErrorInvalidValue;
    if (!x_dev || !xs_dev || !w_planes_dev || !ws_dev || !y_dev || !os_dev ||
        ws_bytes < kt_hip_quant_linear_workspace(rows, in_f, out_f, nullptr))
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_quant_linear(x_dev, rows, in_f, xs_dev, w_planes_dev, pw, out_f, w_mant, w_shift, bias_dev,
                                        b_mant, b_shift, flush_of(3, pw), ws_dev, y_dev, os_dev,
                                        (hipStream_t)stream);
}

int kt_hip_quant_linear_multi(int dev, const int32_t* x_dev, int64_t rows, int64_t in_f, const kt_hip_qscale* xs_dev,
                              int nseg, const int64_t* seg_out, const int8_t* w_planes_dev, int pw,
                              const int64_t* w_mant, const int32_t* w_shift, const int64_t* bias_dev,
                              const int* has_bias, const int64_t* b_mant, const int32_t* b_shift, void* ws_dev,
                              size_t ws_bytes, int32_t* const* y_devs, kt_hip_qscale* os_dev, void* stream) {
    if (nseg < 1 || nseg > KT_QL_MAX_SEGMENTS || !seg_out || !w_mant || !w_shift || !y_devs || rows < 1 ||
        in_f < 1 || (pw != 1 && pw != 3 && pw != 5) || (bias_dev && (!has_bias || !b_mant || !b_shift)))
        return (int)hipErrorInvalidValue;
    int64_t out_f = 0;
    for (int g = 0; g < nseg; g++) {
        if (seg_out[g] < 1 || w_mant[g] < 0 || (bias_dev && has_bias[g] && b_mant[g] < 0) || !y_devs[g])
            return (int)hipErrorInvalidValue;
        out_f += seg_out[g];
    }
    const int64_t kp = kp_of(in_f);
    if (rows * kp >= ((int64_t)1 << 31) || rows * out_f >= ((int64_t)1 << 31) || kp > INT_MAX)
        return (int)hipErrorInvalidValue;
    if (!x_dev || !xs_dev || !w_planes_dev || !ws_dev || !os_dev ||
        ws_bytes < kt_hip_quant_linear_workspace(rows, in_f, out_f, nullptr))
        return (int)hipErrorInvalidValue;
    // every CTA of the digit GEMM covers columns of one call: each boundary a multiple of its CTA's columns
    const int64_t cols = kt::plane_gemm_cta_cols(3, pw, (int)rows, (int)out_f);
    for (int64_t g = 0, at = 0; g + 1 < nseg; g++)
        if ((at += seg_out[g]) % cols) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_quant_linear_multi(x_dev, rows, in_f, xs_dev, w_planes_dev, pw, nseg, seg_out, w_mant,
                                              w_shift, bias_dev, has_bias, b_mant, b_shift, flush_of(3, pw), ws_dev,
                                              y_devs, os_dev, (hipStream_t)stream);
}

int kt_hip_quant_linear_sums_ok(int64_t in_f, int64_t out_f, int pw) {
    if (pw != 1 && pw != 3 && pw != 5) return 0;
    return kt::ql_sums_ok(in_f, out_f, pw, flush_of(3, pw)) ? 1 : 0;
}

int kt_hip_quant_linear_multi_sums(int dev, const int32_t* x_dev, int64_t in_f, const kt_hip_qscale* xs_dev,
                                   int nseg, const int64_t* seg_out, const int8_t* w_planes_dev, int pw,
                                   const int64_t* w_mant, const int32_t* w_shift, void* ws_dev, size_t ws_bytes,
                                   void* stream) {
    if (nseg < 1 || nseg > KT_QL_MAX_SEGMENTS || !seg_out || !w_mant || !w_shift || in_f < 1 ||
        (pw != 1 && pw != 3 && pw != 5))
        return (int)hipErrorInvalidValue;
    int64_t out_f = 0;
    for (int g = 0; g < nseg; g++) {
        if (seg_out[g] < 1 || w_mant[g] < 0 || (g + 1 < nseg && (out_f + seg_out[g]) % 8))
            return (int)hipErrorInvalidValue;
        out_f += seg_out[g];
    }
    if (!kt_hip_quant_linear_sums_ok(in_f, out_f, pw) || !x_dev || !xs_dev || !w_planes_dev || !ws_dev ||
        ws_bytes < kt_hip_quant_linear_workspace(1, in_f, out_f, nullptr))
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_quant_linear_sums(x_dev, in_f, xs_dev, w_planes_dev, pw, nseg, seg_out, w_mant, w_shift,
                                             flush_of(3, pw), ws_dev, (hipStream_t)stream);
}

int64_t kt_hip_quant_linear_multi_align(int64_t rows, int64_t out_f, int pw) {
    if (rows < 1 || out_f < 1 || rows > INT_MAX || out_f > INT_MAX || (pw != 1 && pw != 3 && pw != 5)) return 0;
    return kt::plane_gemm_cta_cols(3, pw, (int)rows, (int)out_f);
}

int kt_hip_quant_linear_noalloc(int dev, const int32_t* x_dev, int64_t rows, int64_t in_f,
                                const kt_hip_qscale* xs_dev, const int8_t* w_planes_dev, int pw, int64_t out_f,
                                int64_t w_mant, int32_t w_shift, const int64_t* bias_dev, int64_t b_mant,
                                int32_t b_shift, int32_t* y_dev, kt_hip_qscale* os_dev, void* stream) {
    if (rows < 1 || in_f < 1 || out_f < 1 || (pw != 1 && pw != 3 && pw != 5) || w_mant < 0 || b_mant < 0)
        return (int)hipErrorInvalidValue;
    const int64_t kp = kp_of(in_f);
    if (rows * kp >= ((int64_t)1 << 31) || rows * out_f >= ((int64_t)1 << 31) || kp > INT_MAX)
        return (int)hipErrorInvalidValue;
    if (!x_dev || !xs_dev || !w_planes_dev || !y_dev || !os_dev) return (int)hipErrorInvalidValue;
    const size_t need = kt_hip_quant_linear_workspace(rows, in_f, out_f, nullptr);
    if (need == 0 || need > KT_QL_SCRATCH_BYTES) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    void* ws = nullptr;
    KT_TRY(kt::ql_scratch(dev, &ws, (hipStream_t)stream));
    return (int)kt::launch_quant_linear(x_dev, rows, in_f, xs_dev, w_planes_dev, pw, out_f, w_mant, w_shift, bias_dev,
                                        b_mant, b_shift, flush_of(3, pw), ws, y_dev, os_dev, (hipStream_t)stream);
}

// ----------------------------------------------------------------------------------------------------------------
// Backend layer (TcLinear, crates/02-runtime/kt-cuda/src/backend.rs:77-192)
// ----------------------------------------------------------------------------------------------------------------

static int open_impl(int dev, uint64_t budget, int plant, kt_hip_backend** out) {
    *out = nullptr;
    int n = 0;
    KT_TRY(hipGetDeviceCount(&n));
    if (dev < 0 || dev >= n) return (int)hipErrorInvalidDevice;
    hipDeviceProp_t p;
    KT_TRY(hipGetDeviceProperties(&p, dev));
    KT_TRY(hipSetDevice(dev));
    size_t free_b = 0, total = 0;
    KT_TRY(hipMemGetInfo(&free_b, &total));
    kt_hip_backend* b = new kt_hip_backend();
    b->dev = dev;
    b->devname = device_name(p);
    b->budget_given = budget != 0;
    b->budget = budget != 0 ? budget : (uint64_t)free_b / 5 * 4;  // kt-cuda/src/device.rs:147-149
    b->plant = plant;
    hipError_t e = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete b;
        return (int)e;
    }
    *out = b;
    return 0;
}

int kt_hip_open(int dev, uint64_t budget_bytes, kt_hip_backend** out) { return open_impl(dev, budget_bytes, 0, out); }

int kt_hip_open_planted(int dev, int plant, kt_hip_backend** out) {
#ifdef KT_HIP_PLANTS
    if (plant < KT_PLANT_DROP_TOP || plant > KT_PLANT_CACHE_BY_SHAPE) return (int)hipErrorInvalidValue;
    return open_impl(dev, 0, plant, out);
#else
    (void)dev;
    (void)plant;
    *out = nullptr;
    return (int)hipErrorNotSupported;  // plants exist only in the test build
#endif
}

void kt_hip_close(kt_hip_backend* b) {
    if (!b) return;
    {
        std::lock_guard<std::mutex> g(b->mu);
        (void)hipSetDevice(b->dev);
        (void)hipStreamSynchronize(b->stream);
        for (auto& kv : b->cache) (void)hipFree(kv.second.planes);
        b->cache.clear();
        b->xcodes.release();
        b->xplanes.release();
        b->ydev.release();
        b->wcodes.release();
        (void)hipStreamDestroy(b->stream);
    }
    delete b;
}

int kt_hip_name(const kt_hip_backend* b, char* buf, int len) {
    std::string s;
    if (b->plant) s = std::string("planted-hip-") + plant_name(b->plant);
    else if (b->budget_given) s = "hip:" + b->devname + " [budget " + std::to_string(b->budget) + " B]";
    else s = "hip:" + b->devname;
    if (len <= 0) return (int)hipErrorInvalidValue;
    strncpy(buf, s.c_str(), (size_t)len - 1);
    buf[len - 1] = 0;
    return 0;
}

uint64_t kt_hip_weight_id_fresh(void) { return g_next_id.fetch_add(1); }

uint64_t kt_hip_resident_bytes(const kt_hip_backend* b) {
    std::lock_guard<std::mutex> g(const_cast<kt_hip_backend*>(b)->mu);
    return b->bytes;
}

uint64_t kt_hip_fallbacks(void) { return g_fallbacks.load(); }

// Packed weights for this call (TcLinear::weights, backend.rs:125-154): resident if the key was seen, else uploaded,
// packed on the device and cached under the budget, evicting the least recently used. A weight larger than the
// budget is used for its call and dropped (*temp = true).
static hipError_t weights_for(kt_hip_backend* b, const int32_t* w, const uint64_t* id, size_t out, size_t k,
                              int8_t** planes, int* pw, bool* temp) {
    const bool keyed = id != nullptr;
    const bool by_id = keyed && b->plant != KT_PLANT_CACHE_BY_SHAPE;  // the planted cache drops the id
    Key key{by_id, by_id ? *id : 0, out, k};
    b->tick++;
    if (keyed) {
        auto it = b->cache.find(key);
        if (it != b->cache.end()) {
            it->second.last_use = b->tick;
            *planes = it->second.planes;
            *pw = it->second.pw;
            *temp = false;
            return hipSuccess;
        }
    }
    const int p = plane_class(digits_for(w, out * k));
    const int64_t kp = kp_of((int64_t)k);
    const uint64_t bytes = (uint64_t)p * out * (uint64_t)kp;
    hipError_t e = b->wcodes.grow(out * k * sizeof(int32_t));
    if (e != hipSuccess) return e;
    e = hipMemcpyAsync(b->wcodes.ptr, w, out * k * sizeof(int32_t), hipMemcpyHostToDevice, b->stream);
    if (e != hipSuccess) return e;
    if (keyed) {
        while (b->bytes + bytes > b->budget && !b->cache.empty()) {
            auto lru = b->cache.begin();
            for (auto it = b->cache.begin(); it != b->cache.end(); ++it)
                if (it->second.last_use < lru->second.last_use) lru = it;
            e = hipStreamSynchronize(b->stream);  // nothing queued may still read the evicted planes
            if (e != hipSuccess) return e;
            e = hipFree(lru->second.planes);
            b->bytes -= lru->second.bytes;
            b->cache.erase(lru);
            if (e != hipSuccess) return e;
        }
    }
    int8_t* dst = nullptr;
    e = hipMalloc((void**)&dst, bytes);
    if (e != hipSuccess) return e;
    e = kt::launch_pack_planes((const int32_t*)b->wcodes.ptr, (int64_t)out, (int64_t)k, p, 0, dst, b->stream);
    if (e != hipSuccess) {
        (void)hipFree(dst);
        return e;
    }
    *planes = dst;
    *pw = p;
    *temp = !(keyed && bytes <= b->budget);
    if (!*temp) {
        b->cache[key] = Entry{dst, p, bytes, b->tick};
        b->bytes += bytes;
    }
    return hipSuccess;
}

// TcLinear::run (backend.rs:156-172) on the device.
static int run(kt_hip_backend* b, const int32_t* x, const int32_t* w, const uint64_t* id, size_t rows, size_t out,
               size_t k, int64_t* y) {
    if (rows == 0 || out == 0) return 0;
    if (k == 0) {
        memset(y, 0, rows * out * sizeof(int64_t));
        return 0;
    }
    const int64_t kp = kp_of((int64_t)k);
    if (rows > INT_MAX || out > INT_MAX || kp > INT_MAX) return (int)hipErrorInvalidValue;
    std::lock_guard<std::mutex> g(b->mu);
    KT_TRY(hipSetDevice(b->dev));
    const int px = plane_class(digits_for(x, rows * k));
    int8_t* wplanes = nullptr;
    int pw = 0;
    bool temp = false;
    KT_TRY(weights_for(b, w, id, out, k, &wplanes, &pw, &temp));
    hipError_t e = hipSuccess;
    auto fail = [&](hipError_t err) {
        if (temp) {
            (void)hipStreamSynchronize(b->stream);
            (void)hipFree(wplanes);
        }
        return (int)err;
    };
    if ((e = b->xcodes.grow(rows * k * sizeof(int32_t))) != hipSuccess) return fail(e);
    if ((e = b->xplanes.grow((size_t)px * rows * (size_t)kp)) != hipSuccess) return fail(e);
    if ((e = b->ydev.grow(rows * out * sizeof(int64_t))) != hipSuccess) return fail(e);
    if ((e = hipMemcpyAsync(b->xcodes.ptr, x, rows * k * sizeof(int32_t), hipMemcpyHostToDevice, b->stream)) !=
        hipSuccess)
        return fail(e);
    const int wrong_carry = b->plant == KT_PLANT_WRONG_CARRY;
    if ((e = kt::launch_pack_planes((const int32_t*)b->xcodes.ptr, (int64_t)rows, (int64_t)k, px, wrong_carry,
                                    (int8_t*)b->xplanes.ptr, b->stream)) != hipSuccess)
        return fail(e);
    const int64_t fk = b->plant == KT_PLANT_NO_FLUSH ? kp : flush_of(px, pw);
    for (int64_t k0 = 0; k0 < kp; k0 += fk) {
        const int64_t k1 = kp - k0 < fk ? kp : k0 + fk;
        if ((e = kt::launch_plane_gemm(px, pw, (const int8_t*)b->xplanes.ptr, wplanes, (int64_t*)b->ydev.ptr,
                                       (int)rows, (int)out, (int)kp, (int)k0, (int)k1, k0 > 0,
                                       b->plant == KT_PLANT_DROP_TOP, b->stream)) != hipSuccess)
            return fail(e);
    }
    if ((e = hipMemcpyAsync(y, b->ydev.ptr, rows * out * sizeof(int64_t), hipMemcpyDeviceToHost, b->stream)) !=
        hipSuccess)
        return fail(e);
    if ((e = hipStreamSynchronize(b->stream)) != hipSuccess) return fail(e);
    if (temp) KT_TRY(hipFree(wplanes));
    return 0;
}

int kt_hip_linear(kt_hip_backend* b, const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k,
                  int64_t* y) {
    return run(b, x, w, nullptr, rows, out, k, y);
}

int kt_hip_linear_weights(kt_hip_backend* b, const int32_t* x, uint64_t weight_id, const int32_t* w, size_t rows,
                          size_t out, size_t k, int64_t* y) {
    return run(b, x, w, &weight_id, rows, out, k, y);
}

// ----------------------------------------------------------------------------------------------------------------
// 12-bit-weight path
// ----------------------------------------------------------------------------------------------------------------

void kt_hip_w12_bytes(int64_t n, int64_t k, size_t* lo_bytes, size_t* nib_bytes) {
    const size_t lo = (size_t)((n + 31) / 32 * 32) * (size_t)kp_of(k);
    *lo_bytes = lo;
    *nib_bytes = lo / 2;
}

int kt_hip_w12_pack(int dev, const int32_t* codes_dev, int64_t n, int64_t k, int8_t* lo_dev, uint8_t* nib_dev,
                    void* stream) {
    if (n < 0 || k < 0) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_w12_pack(codes_dev, n, k, 0, lo_dev, nib_dev, (hipStream_t)stream);
}

int kt_hip_w12_upload(int dev, const int32_t* codes, int64_t n, int64_t k, int8_t* lo_dev, uint8_t* nib_dev) {
    if (n < 0 || k < 0) return (int)hipErrorInvalidValue;
    const size_t cnt = (size_t)n * (size_t)k;
    for (size_t i = 0; i < cnt; i++)
        if (codes[i] < -2048 || codes[i] > 2047) return (int)hipErrorInvalidValue;
    if (cnt == 0) return 0;
    KT_TRY(hipSetDevice(dev));
    void* tmp = nullptr;
    KT_TRY(hipMalloc(&tmp, cnt * sizeof(int32_t)));
    hipError_t e = hipMemcpy(tmp, codes, cnt * sizeof(int32_t), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = kt::launch_w12_pack((const int32_t*)tmp, n, k, 0, lo_dev, nib_dev, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    hipError_t f = hipFree(tmp);
    return (int)(e != hipSuccess ? e : f);
}

int kt_hip_w12_linear(int dev, const int8_t* x_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                      int64_t n, int64_t k, const int32_t* mant_dev, const int32_t* shift_dev, int out_kind,
                      void* y_dev, void* stream) {
    if (m < 0 || n < 0 || k < 0) return (int)hipErrorInvalidValue;
    if (m == 0 || n == 0) return 0;
    const int64_t kp = kp_of(k);
    if (m > INT_MAX || n > INT_MAX || kp > INT_MAX) return (int)hipErrorInvalidValue;
    if (out_kind != KT_OUT_I64 && (mant_dev == nullptr || shift_dev == nullptr)) return (int)hipErrorInvalidValue;
    if (out_kind != KT_OUT_I64 && out_kind != KT_OUT_I32 && out_kind != KT_OUT_I8 && out_kind != KT_OUT_I32_ADD)
        return (int)hipErrorInvalidValue;
    if (kp > (m > KT_W12_SKINNY_MAX_M ? KT_W12_GEMM_MAX_K : KT_W12_SKINNY_MAX_K)) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    if (kp == 0) {
        // an empty dot is 0; its requant is 0 as well (and adds nothing)
        if (out_kind == KT_OUT_I32_ADD) return 0;
        const size_t w = out_kind == KT_OUT_I64 ? 8 : (out_kind == KT_OUT_I32 ? 4 : 1);
        return (int)hipMemsetAsync(y_dev, 0, (size_t)m * (size_t)n * w, (hipStream_t)stream);
    }
    return (int)kt::launch_w12_linear(x_dev, lo_dev, nib_dev, (int)m, (int)n, (int)kp, mant_dev, shift_dev, nullptr, out_kind,
                                      y_dev, (hipStream_t)stream);
}

void kt_hip_w12b_bytes(int64_t n, int64_t k, size_t* plane_bytes) {
    *plane_bytes = (size_t)((n + 31) / 32 * 32) * (size_t)kp_of(k);
}

int kt_hip_w12b_pack(int dev, const int32_t* codes_dev, int64_t n, int64_t k, int8_t* lo_dev, int8_t* hi_dev,
                     void* stream) {
    if (n < 0 || k < 0) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_w12b_pack(codes_dev, n, k, lo_dev, hi_dev, (hipStream_t)stream);
}

int kt_hip_w12b_linear(int dev, const int8_t* x_dev, const int8_t* lo_dev, const int8_t* hi_dev, int64_t m,
                       int64_t n, int64_t k, const int32_t* mant_dev, const int32_t* shift_dev, int out_kind,
                       void* y_dev, void* stream) {
    if (m < 0 || n < 0 || k < 1) return (int)hipErrorInvalidValue;
    if (m == 0 || n == 0) return 0;
    const int64_t kp = kp_of(k);
    if (m > INT_MAX || n > INT_MAX || kp > KT_W12_GEMM_MAX_K) return (int)hipErrorInvalidValue;
    if (m * kp > (int64_t)UINT32_MAX || (n + 31) / 32 * 32 * kp > (int64_t)UINT32_MAX) return (int)hipErrorInvalidValue;
    if (out_kind != KT_OUT_I64 && (mant_dev == nullptr || shift_dev == nullptr)) return (int)hipErrorInvalidValue;
    if (out_kind != KT_OUT_I64 && out_kind != KT_OUT_I32 && out_kind != KT_OUT_I8 && out_kind != KT_OUT_I32_ADD)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_w12b_linear(x_dev, lo_dev, hi_dev, (int)m, (int)n, (int)kp, mant_dev, shift_dev, out_kind,
                                       y_dev, (hipStream_t)stream);
}

int kt_hip_stream_read(int dev, const uint8_t* src_dev, int64_t bytes_n, uint32_t* out_dev, void* stream) {
    if (bytes_n < 0 || bytes_n % 16 || bytes_n >= ((int64_t)1 << 31) || out_dev == nullptr ||
        (bytes_n > 0 && src_dev == nullptr))
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_stream_read(src_dev, (uint32_t)bytes_n, out_dev, (hipStream_t)stream);
}

int kt_hip_w12_linear_lut(int dev, const int8_t* x_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                          int64_t n, int64_t k, const int32_t* mant_dev, const int32_t* shift_dev,
                          const int8_t* lut_dev, int8_t* y_dev, void* stream) {
    if (m < 0 || n < 0 || k < 1 || lut_dev == nullptr || mant_dev == nullptr || shift_dev == nullptr)
        return (int)hipErrorInvalidValue;
    if (m == 0 || n == 0) return 0;
    const int64_t kp = kp_of(k);
    if (m > INT_MAX || n > INT_MAX || kp > 8128) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_w12_linear(x_dev, lo_dev, nib_dev, (int)m, (int)n, (int)kp, mant_dev, shift_dev, lut_dev,
                                      KT_OUT_I8, y_dev, (hipStream_t)stream);
}

// ----------------------------------------------------------------------------------------------------------------
// MoE layer (config 4)
// ----------------------------------------------------------------------------------------------------------------

int kt_hip_w12_pack_gate_up(int dev, const int32_t* codes_dev, int64_t ffn, int64_t k, int8_t* lo_dev,
                            uint8_t* nib_dev, void* stream) {
    if (ffn <= 0 || k < 0 || ffn % 32) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_w12_pack(codes_dev, 2 * ffn, k, ffn, lo_dev, nib_dev, (hipStream_t)stream);
}

int kt_hip_moe_route(int dev, const int32_t* logits_dev, int64_t tokens, int64_t experts, int top_k,
                     const int16_t* sig_dev, int32_t* sel_dev, int32_t* cw_dev, void* stream) {
    if (tokens < 0 || tokens > INT_MAX / 64 || experts < 1 || experts > 1024) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_moe_route(logits_dev, (int)tokens, (int)experts, top_k, sig_dev, sel_dev, cw_dev,
                                     (hipStream_t)stream);
}

int kt_hip_moe_bucket(int dev, const int32_t* sel_dev, int64_t tokens, int64_t experts, int top_k,
                      int32_t* list_dev, int32_t* pos_dev, int32_t* count_dev, void* stream) {
    if (tokens < 0 || experts < 1 || (experts + 1) * tokens > INT_MAX || tokens * top_k > INT_MAX)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_moe_bucket(sel_dev, (int)tokens, (int)experts, top_k, list_dev, pos_dev, count_dev,
                                      (hipStream_t)stream);
}

int kt_hip_w12_grouped_linear(int dev, const int8_t* x_dev, int64_t x_rows, const int32_t* list_dev,
                              int64_t list_stride, const int32_t* count_dev, int64_t groups, int64_t max_rows,
                              const int8_t* lo_dev, const uint8_t* nib_dev, int64_t n, int64_t k,
                              const int32_t* mant_dev, const int32_t* shift_dev, int epilogue,
                              const int16_t* silu_dev, int h_shift, int8_t* y_dev, int64_t y_stride,
                              int32_t* off_dev, void* stream) {
    if (x_rows < 0 || groups < 0 || max_rows < 0 || n < 0 || k < 1 || y_stride < 0 || list_stride < 0)
        return (int)hipErrorInvalidValue;
    if (groups == 0 || n == 0) return 0;
    const int64_t kp = kp_of(k);
    if (groups > KT_MAX_GROUPS || kp > 8128 || n > INT_MAX || y_stride > INT_MAX || list_stride > INT_MAX ||
        mant_dev == nullptr || shift_dev == nullptr)
        return (int)hipErrorInvalidValue;
    const int64_t ycols = epilogue == KT_EPI_SWIGLU ? n / 2 : n;
    if (y_stride < ycols) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    size_t lo_bytes = 0, nib_bytes = 0;
    kt_hip_w12_bytes(n, k, &lo_bytes, &nib_bytes);
    return (int)kt::launch_w12_grouped(x_dev, (size_t)x_rows * (size_t)kp, list_dev, (int)list_stride, count_dev,
                                       (int)groups, max_rows, lo_dev, nib_dev, lo_bytes, (int)n, (int)kp, mant_dev,
                                       shift_dev, epilogue, silu_dev, h_shift, y_dev, (int)y_stride, off_dev,
                                       (hipStream_t)stream);
}

int kt_hip_w12_swiglu(int dev, const int8_t* x_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                      int64_t ffn, int64_t k, const int32_t* mant_dev, const int32_t* shift_dev,
                      const int16_t* silu_dev, int h_shift, int8_t* y_dev, int64_t y_stride, void* stream) {
    if (m < 0 || ffn <= 0 || ffn % 64 || k < 1 || kp_of(k) > 8128 || y_stride < ffn || y_stride > INT_MAX ||
        m > INT_MAX || mant_dev == nullptr || shift_dev == nullptr || silu_dev == nullptr || h_shift < 1 ||
        h_shift > 30)
        return (int)hipErrorInvalidValue;
    if (m == 0) return 0;
    const int64_t kp = kp_of(k);
    KT_TRY(hipSetDevice(dev));
    if (m <= KT_W12_SKINNY_MAX_M)
        return (int)kt::launch_w12_swiglu(x_dev, lo_dev, nib_dev, (int)m, (int)ffn, (int)kp, mant_dev, shift_dev,
                                          silu_dev, h_shift, y_dev, (int)y_stride, (hipStream_t)stream);
    size_t lo_bytes = 0, nib_bytes = 0;
    kt_hip_w12_bytes(2 * ffn, k, &lo_bytes, &nib_bytes);
    return (int)kt::launch_w12_grouped(x_dev, (size_t)m * (size_t)kp, nullptr, 0, nullptr, 1, m, lo_dev, nib_dev,
                                       lo_bytes, (int)(2 * ffn), (int)kp, mant_dev, shift_dev, KT_EPI_SWIGLU,
                                       silu_dev, h_shift, y_dev, (int)y_stride, nullptr, (hipStream_t)stream);
}

int kt_hip_w12_linear_norm(int dev, const int32_t* r_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                           int64_t n, int64_t d, const int32_t* mant_dev, const int32_t* shift_dev, int out_kind,
                           void* y_dev, void* stream) {
    if (m < 1 || m > KT_NORM_MAX_M || n < 1 || n > INT_MAX || d < 1 || kp_of(d) > KT_NORM_MAX_D ||
        m * kp_of(d) > KT_NORM_LDS_BYTES || r_dev == nullptr || y_dev == nullptr || y_dev == (void*)r_dev ||
        (out_kind != KT_OUT_I64 && out_kind != KT_OUT_I32 && out_kind != KT_OUT_I8) ||
        (out_kind != KT_OUT_I64 && (mant_dev == nullptr || shift_dev == nullptr)))
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_w12_linear_norm(r_dev, (int)m, (int)d, lo_dev, nib_dev, (int)n, mant_dev, shift_dev,
                                           out_kind, y_dev, (hipStream_t)stream);
}

int kt_hip_w12_swiglu_norm(int dev, const int32_t* r_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                           int64_t ffn, int64_t d, const int32_t* mant_dev, const int32_t* shift_dev,
                           const int16_t* silu_dev, int h_shift, int8_t* y_dev, int64_t y_stride, void* stream) {
    if (m < 1 || m > KT_NORM_MAX_M || ffn <= 0 || ffn % 64 || ffn > INT_MAX || d < 1 || kp_of(d) > KT_NORM_MAX_D ||
        m * kp_of(d) > KT_NORM_LDS_BYTES || y_stride < ffn || y_stride > INT_MAX || r_dev == nullptr ||
        mant_dev == nullptr || shift_dev == nullptr || silu_dev == nullptr || h_shift < 1 || h_shift > 30)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_w12_swiglu_norm(r_dev, (int)m, (int)d, lo_dev, nib_dev, (int)ffn, mant_dev, shift_dev,
                                           silu_dev, h_shift, y_dev, (int)y_stride, (hipStream_t)stream);
}

int kt_hip_moe_combine(int dev, const int8_t* d_dev, const int32_t* off_dev, const int32_t* sel_dev,
                       const int32_t* cw_dev, const int32_t* pos_dev, int64_t tokens, int64_t hidden,
                       int64_t experts, int top_k, int out_shift, int8_t* out_dev, void* stream) {
    if (tokens < 0 || tokens > INT_MAX || hidden < 0 || hidden > INT_MAX || experts < 1) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_moe_combine(d_dev, off_dev, sel_dev, cw_dev, pos_dev, (int)tokens, (int)hidden,
                                       (int)experts, top_k, out_shift, out_dev, (hipStream_t)stream);
}

static size_t align256(size_t v) { return (v + 255) / 256 * 256; }

int kt_hip_moe_workspace(int64_t tokens, int64_t hidden, int64_t ffn, int64_t experts, int top_k, size_t* total,
                         size_t* offsets) {
    if (tokens < 0 || hidden < 0 || ffn < 0 || experts < 1 || top_k < 1) return (int)hipErrorInvalidValue;
    const size_t T = (size_t)tokens, E = (size_t)experts, K = (size_t)top_k, P = T * (K + 1);
    const size_t sizes[KT_MOE_WS_PARTS] = {T * K * 4, T * K * 4, T * K * 4, (E + 1) * T * 4,
                                           (E + 1) * 4, (E + 2) * 4, P * (size_t)ffn, P * (size_t)hidden};
    size_t at = 0;
    for (int i = 0; i < KT_MOE_WS_PARTS; i++) {
        if (offsets) offsets[i] = at;
        at += align256(sizes[i]);
    }
    *total = at;
    return 0;
}

int kt_hip_moe_forward(int dev, const int8_t* x_dev, const int32_t* logits_dev, int64_t tokens, int64_t hidden,
                       int64_t ffn, int64_t experts, int top_k, const int8_t* gu_lo_dev, const uint8_t* gu_nib_dev,
                       const int32_t* gu_mant_dev, const int32_t* gu_shift_dev, const int8_t* d_lo_dev,
                       const uint8_t* d_nib_dev, const int32_t* d_mant_dev, const int32_t* d_shift_dev,
                       const int16_t* silu_dev, const int16_t* sig_dev, int h_shift, int out_shift,
                       void* workspace_dev, int8_t* out_dev, void* stream) {
    if (tokens < 0 || hidden <= 0 || ffn <= 0 || hidden % 64 || ffn % 64 || hidden > 8128 || ffn > 8128 ||
        experts < 1 || experts + 1 > KT_MAX_GROUPS || top_k < 1 || top_k > experts || top_k > 32 ||
        workspace_dev == nullptr)
        return (int)hipErrorInvalidValue;
    if (tokens == 0) return 0;
    const int64_t P = tokens * (top_k + 1);
    if (P * hidden > (int64_t)0xFFFFFF00 || tokens * hidden > (int64_t)0xFFFFFF00 || (experts + 1) * tokens > INT_MAX)
        return (int)hipErrorInvalidValue;
    size_t total = 0, off[KT_MOE_WS_PARTS];
    KT_TRY((hipError_t)kt_hip_moe_workspace(tokens, hidden, ffn, experts, top_k, &total, off));
    char* ws = (char*)workspace_dev;
    int32_t *sel = (int32_t*)(ws + off[0]), *cw = (int32_t*)(ws + off[1]), *pos = (int32_t*)(ws + off[2]);
    int32_t *list = (int32_t*)(ws + off[3]), *count = (int32_t*)(ws + off[4]), *goff = (int32_t*)(ws + off[5]);
    int8_t *h = (int8_t*)(ws + off[6]), *d = (int8_t*)(ws + off[7]);
    hipStream_t s = (hipStream_t)stream;
    KT_TRY(hipSetDevice(dev));
    const int T = (int)tokens, E = (int)experts;
    KT_TRY(kt::launch_moe_route(logits_dev, T, E, top_k, sig_dev, sel, cw, s));
    KT_TRY(kt::launch_moe_bucket(sel, T, E, top_k, list, pos, count, s));
    size_t gu_lo = 0, gu_nib = 0, dn_lo = 0, dn_nib = 0;
    kt_hip_w12_bytes(2 * ffn, hidden, &gu_lo, &gu_nib);
    kt_hip_w12_bytes(hidden, ffn, &dn_lo, &dn_nib);
    KT_TRY(kt::launch_w12_grouped(x_dev, (size_t)tokens * (size_t)hidden, list, T, count, E + 1, P, gu_lo_dev,
                                  gu_nib_dev, gu_lo, (int)(2 * ffn), (int)hidden, gu_mant_dev, gu_shift_dev,
                                  KT_EPI_SWIGLU, silu_dev, h_shift, h, (int)ffn, goff, s));
    KT_TRY(kt::launch_w12_grouped(h, (size_t)P * (size_t)ffn, nullptr, 0, count, E + 1, P, d_lo_dev, d_nib_dev, dn_lo,
                                  (int)hidden, (int)ffn, d_mant_dev, d_shift_dev, KT_EPI_I8, nullptr, 0, d,
                                  (int)hidden, nullptr, s));
    return (int)kt::launch_moe_combine(d, goff, sel, cw, pos, T, (int)hidden, E, top_k, out_shift, out_dev, s);
}

// ----------------------------------------------------------------------------------------------------------------
// SAM image path (config 5)
// ----------------------------------------------------------------------------------------------------------------

// The tap-padded k of a patch-embed weight matrix, 0 for shapes the patch embed does not take.
static int64_t sam_patch_kp(int64_t ci, int64_t kh, int64_t kw) {
    const int kwp = kt::conv_patch_kwp(kw);
    if (ci < 1 || ci > 4 || kh < 1 || kh > 256 || kwp == 0) return 0;
    return ci * kh * kwp;
}

void kt_hip_sam_patch_bytes(int64_t co, int64_t ci, int64_t kh, int64_t kw, size_t* lo_bytes, size_t* hi_bytes) {
    const int64_t k = sam_patch_kp(ci, kh, kw);
    if (co < 0 || k == 0) {
        *lo_bytes = *hi_bytes = 0;
        return;
    }
    *lo_bytes = *hi_bytes = (size_t)((co + 31) / 32 * 32) * (size_t)kp_of(k);
}

int kt_hip_sam_patch_pack(int dev, const int32_t* codes_dev, int64_t co, int64_t ci, int64_t kh, int64_t kw,
                          int8_t* lo_dev, int8_t* hi_dev, void* stream) {
    if (co < 0 || co > INT_MAX / 2 || sam_patch_kp(ci, kh, kw) == 0) return (int)hipErrorInvalidValue;
    if (co == 0) return 0;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_conv_pack(codes_dev, (int)co, (int)ci, (int)kh, (int)kw, lo_dev, hi_dev,
                                     (hipStream_t)stream);
}

int kt_hip_sam_patch_upload(int dev, const int32_t* codes, int64_t co, int64_t ci, int64_t kh, int64_t kw,
                            int8_t* lo_dev, int8_t* hi_dev) {
    if (co < 0 || co > INT_MAX / 2 || sam_patch_kp(ci, kh, kw) == 0) return (int)hipErrorInvalidValue;
    const size_t cnt = (size_t)co * (size_t)(ci * kh * kw);
    for (size_t i = 0; i < cnt; i++)
        if (codes[i] < -2048 || codes[i] > 2047) return (int)hipErrorInvalidValue;
    if (cnt == 0) return 0;
    KT_TRY(hipSetDevice(dev));
    void* tmp = nullptr;
    KT_TRY(hipMalloc(&tmp, cnt * sizeof(int32_t)));
    hipError_t e = hipMemcpy(tmp, codes, cnt * sizeof(int32_t), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = kt::launch_conv_pack((const int32_t*)tmp, (int)co, (int)ci, (int)kh, (int)kw, lo_dev, hi_dev, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    hipError_t f = hipFree(tmp);
    return (int)(e != hipSuccess ? e : f);
}

int kt_hip_sam_patch_embed(int dev, const uint8_t* img_dev, const int8_t* lut_dev, int64_t ci, int64_t h, int64_t w,
                           const int8_t* lo_dev, const int8_t* hi_dev, int64_t co, int64_t kh, int64_t kw,
                           int64_t stride, int64_t pad, const int32_t* bias_dev, const int32_t* mant_dev,
                           const int32_t* shift_dev, int8_t* out_dev, void* stream) {
    if (ci < 1 || ci > 4 || h < 1 || w < 1 || h > INT_MAX || w > INT_MAX || co < 1 || co > INT_MAX || kh < 1 ||
        kw < 1 || kh > 256 || kw > 256 || stride < 1 || stride > 256 || pad < 0 || pad > 256 || mant_dev == nullptr ||
        shift_dev == nullptr || lut_dev == nullptr)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_conv_patch(img_dev, lut_dev, (int)ci, (int)h, (int)w, (int)kh, (int)kw, (int)stride,
                                      (int)pad, lo_dev, hi_dev, (int)co, bias_dev, mant_dev, shift_dev, out_dev,
                                      (hipStream_t)stream);
}

// ----------------------------------------------------------------------------------------------------------------
// Decoder (config 3)
// ----------------------------------------------------------------------------------------------------------------

int kt_hip_dec_embed(int dev, const int32_t* tokens_dev, int64_t tokens, const int16_t* emb_dev, int64_t d,
                     int32_t* r_dev, void* stream) {
    if (tokens < 0 || tokens > INT_MAX || d < 1 || d > INT_MAX) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_embed(tokens_dev, (int)tokens, emb_dev, (int)d, r_dev, (hipStream_t)stream);
}

int kt_hip_dec_rmsnorm(int dev, const int32_t* r_dev, int64_t tokens, int64_t d, int8_t* q_dev, int64_t q_stride,
                       void* stream) {
    if (tokens < 0 || tokens > INT_MAX || d < 1 || d > (1 << 20) || q_stride < d || q_stride > INT_MAX)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_rmsnorm(r_dev, (int)tokens, (int)d, q_dev, (int)q_stride, (hipStream_t)stream);
}

int kt_hip_dec_rope_kv(int dev, int8_t* qkv_dev, int64_t tokens, int64_t nqkv, const int32_t* pos_dev, int64_t nh,
                       int64_t nkv, int64_t hd, const int16_t* cos_dev, const int16_t* sin_dev, int8_t* kcache_dev,
                       int8_t* vcache_dev, void* stream) {
    if (tokens < 0 || tokens > INT_MAX || nh < 1 || nkv < 1 || hd < 2 || hd % 2 || nh % nkv ||
        nqkv != (nh + 2 * nkv) * hd || nqkv > INT_MAX)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_rope_kv(qkv_dev, (int)tokens, (int)nqkv, pos_dev, (int)nh, (int)nkv, (int)hd, cos_dev,
                                       sin_dev, kcache_dev, vcache_dev, (hipStream_t)stream);
}

int kt_hip_dec_attention(int dev, const int8_t* qkv_dev, int64_t tokens, int64_t nqkv, const int32_t* pos_dev,
                         const int8_t* kcache_dev, const int8_t* vcache_dev, int64_t nh, int64_t nkv, int64_t hd,
                         const int32_t* exp_tab_dev, int8_t* o_dev, int64_t max_pos, void* stream) {
    if (tokens < 0 || hd != 64 || nh < 1 || nkv < 1 || nh % nkv || nqkv != (nh + 2 * nkv) * hd || max_pos < 1 ||
        max_pos > 16384 || tokens * nh > INT_MAX)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_attention(qkv_dev, (int)tokens, (int)nqkv, pos_dev, kcache_dev, vcache_dev, (int)nh,
                                         (int)nkv, exp_tab_dev, o_dev, (int)max_pos, (hipStream_t)stream);
}

int kt_hip_dec_argmax(int dev, const int32_t* logits_dev, int64_t n, int32_t* token_dev, int32_t* record_dev,
                      int32_t* step_dev, void* stream) {
    if (n < 1 || n > INT_MAX || (record_dev != nullptr && step_dev == nullptr)) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_argmax(logits_dev, (int)n, token_dev, record_dev, step_dev, (hipStream_t)stream);
}

int kt_hip_dec_advance(int dev, int32_t* pos_dev, int64_t by, void* stream) {
    if (by < 0 || by > INT_MAX) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_advance(pos_dev, (int)by, (hipStream_t)stream);
}

int kt_hip_dec_attention_step(int dev, const int8_t* qkv_dev, const int32_t* pos_dev, int8_t* kcache_dev,
                              int8_t* vcache_dev, int64_t nh, int64_t nkv, int64_t hd, const int16_t* cos_dev,
                              const int16_t* sin_dev, const int32_t* exp_tab_dev, int8_t* o_dev, int64_t max_pos,
                              void* stream) {
    if (hd != 64 || nh < 1 || nkv < 1 || nh % nkv || nh > INT_MAX || max_pos < 1 || max_pos > 16384)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_attention_step(qkv_dev, pos_dev, kcache_dev, vcache_dev, (int)nh, (int)nkv, cos_dev,
                                              sin_dev, exp_tab_dev, o_dev, (int)max_pos, (hipStream_t)stream);
}

int kt_hip_dec_attention_o_step(int dev, const int8_t* qkv_dev, const int32_t* pos_dev, int8_t* kcache_dev,
                                int8_t* vcache_dev, int64_t nh, int64_t nkv, int64_t hd, const int16_t* cos_dev,
                                const int16_t* sin_dev, const int32_t* exp_tab_dev, int64_t max_pos,
                                const int8_t* wo_lo_dev, const uint8_t* wo_nib_dev, int64_t d, int32_t* oacc_dev,
                                void* stream) {
    if (hd != 64 || nh < 1 || nkv < 1 || nh % nkv || nh * hd > 8128 || max_pos < 1 || max_pos > 16384 || d < 1 ||
        d > 1024 || !wo_lo_dev || !wo_nib_dev || !oacc_dev)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_attention_o_step(qkv_dev, pos_dev, kcache_dev, vcache_dev, (int)nh, (int)nkv, cos_dev,
                                                sin_dev, exp_tab_dev, (int)max_pos, wo_lo_dev, wo_nib_dev, (int)d,
                                                oacc_dev, (hipStream_t)stream);
}

int kt_hip_w12_swiglu_norm_o(int dev, const int32_t* r_dev, const int8_t* lo_dev, const uint8_t* nib_dev,
                             int64_t ffn, int64_t d, const int32_t* mant_dev, const int32_t* shift_dev,
                             const int16_t* silu_dev, int h_shift, int8_t* y_dev, const int32_t* oacc_dev,
                             const int32_t* omant_dev, const int32_t* oshift_dev, void* stream) {
    if (ffn <= 0 || ffn % 64 || ffn > INT_MAX || d < 1 || d > 1024 || r_dev == nullptr || mant_dev == nullptr ||
        shift_dev == nullptr || silu_dev == nullptr || h_shift < 1 || h_shift > 30 || oacc_dev == nullptr ||
        omant_dev == nullptr || oshift_dev == nullptr)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_w12_swiglu_norm_o(r_dev, (int)d, lo_dev, nib_dev, (int)ffn, mant_dev, shift_dev, silu_dev,
                                             h_shift, y_dev, oacc_dev, omant_dev, oshift_dev, (hipStream_t)stream);
}

int kt_hip_w12_linear_add_o(int dev, const int8_t* x_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t n,
                            int64_t k, const int32_t* mant_dev, const int32_t* shift_dev, int32_t* y_dev,
                            int32_t* oacc_dev, const int32_t* omant_dev, const int32_t* oshift_dev, void* stream) {
    if (n < 1 || n > INT_MAX || k < 1 || kp_of(k) > 8128 || mant_dev == nullptr || shift_dev == nullptr ||
        y_dev == nullptr || oacc_dev == nullptr || omant_dev == nullptr || oshift_dev == nullptr)
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_w12_linear_add_o(x_dev, lo_dev, nib_dev, (int)n, (int)kp_of(k), mant_dev, shift_dev, y_dev,
                                            oacc_dev, omant_dev, oshift_dev, (hipStream_t)stream);
}

int kt_hip_dec_argmax_part(int dev, const int32_t* logits_dev, int64_t n, uint64_t* part_dev, int64_t nparts,
                           int32_t* record_dev, const int32_t* step_dev, int32_t* pos_dev, int64_t advance,
                           void* stream) {
    if (n < 1 || n > INT_MAX || nparts < 1 || nparts > 4096 || nparts > n || advance < 0 || advance > INT_MAX ||
        (record_dev != nullptr && step_dev == nullptr))
        return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_argmax_part(logits_dev, (int)n, part_dev, (int)nparts, record_dev, step_dev, pos_dev,
                                           (int)advance, (hipStream_t)stream);
}

int kt_hip_dec_embed_argmax(int dev, const uint64_t* part_dev, int64_t nparts, const int16_t* emb_dev, int64_t d,
                            int32_t* r_dev, int32_t* token_dev, int32_t* step_dev, void* stream) {
    if (nparts < 1 || nparts > 4096 || d < 1 || d > INT_MAX) return (int)hipErrorInvalidValue;
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_dec_embed_argmax(part_dev, (int)nparts, emb_dev, (int)d, r_dev, token_dev, step_dev,
                                            (hipStream_t)stream);
}

int kt_hip_probe_mfma(int dev, const int8_t* a_dev, const int8_t* b_dev, int32_t* c32_dev, int32_t* c16_dev,
                      void* stream) {
    KT_TRY(hipSetDevice(dev));
    return (int)kt::launch_mfma_probe(a_dev, b_dev, c32_dev, c16_dev, (hipStream_t)stream);
}

}  // extern "C"
