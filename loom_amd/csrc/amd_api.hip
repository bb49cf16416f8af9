// amd_api.hip -- device-resident loom_amd_* entry points (include/loom_accel_amd.h).
#include "api_util.hpp"
#include "lamd.hpp"
#include "loom_accel_amd.h"

#include <string.h>

#include <math.h>

#include <algorithm>
#include <atomic>
#include <memory>
#include <mutex>
#include <thread>
#include <string>
#include <vector>

namespace lamd {

thread_local std::string g_amd_error;

bool is_gfx950(int dev) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return false;
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0;
}

int visible_gfx950() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    int c = 0;
    for (int d = 0; d < n; ++d) c += is_gfx950(d) ? 1 : 0;
    return c;
}

// ---- per-device serialization of the plugin's calls ----------------------

// One lock per device (devices beyond kMaxLockedDevices share the last one).
// The v2 plugin's infer calls hold it from the upload to the stream sync, so
// two host threads running compiled layers on one device never share the
// device's scratch arena and split-K workspace at the same time.
constexpr int kMaxLockedDevices = 64;
static std::mutex g_device_mu[kMaxLockedDevices];

std::mutex& device_mutex(int device) {
    if (device < 0) device = 0;
    if (device >= kMaxLockedDevices) device = kMaxLockedDevices - 1;
    return g_device_mu[device];
}

// ---- per-device scratch arena ------------------------------------------

struct Arena {
    void* ptr = nullptr;
    size_t bytes = 0;
};
static std::mutex g_arena_mu;
static std::vector<Arena> g_arenas;

void* scratch(int device, size_t bytes, std::string* err) {
    std::lock_guard<std::mutex> lock(g_arena_mu);
    if ((int)g_arenas.size() <= device) g_arenas.resize(device + 1);
    Arena& a = g_arenas[device];
    if (a.bytes >= bytes) return a.ptr;
    DeviceGuard guard(device);
    if (a.ptr) {
        // Kernels queued on any stream may still read the old block.
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            *err = std::string("scratch: hipDeviceSynchronize: ") + hipGetErrorString(e);
            return nullptr;
        }
        (void)hipFree(a.ptr);
        a.ptr = nullptr;
        a.bytes = 0;
    }
    size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    want = (want + 4095) & ~(size_t)4095;
    hipError_t e = hipMalloc(&a.ptr, want);
    if (e != hipSuccess) {
        a.ptr = nullptr;
        *err = std::string("scratch: hipMalloc: ") + hipGetErrorString(e);
        return nullptr;
    }
    a.bytes = want;
    return a.ptr;
}

static int ld_for(int k) { return pad_cols(k); }

static int check_matrix(const loom_amd_matrix* w, const char* name) {
    if (w == nullptr || w->m.tiles == nullptr) {
        return fail(std::string(name) + " matrix is null");
    }
    return 0;
}

// The matmul kernels address the tile buffer with 32-bit buffer offsets.
static bool tiles_fit(int rows, int cols) {
    const size_t bytes = (size_t)ceil_div(rows, kTileRows) * (size_t)ceil_div(cols, kTileCols) * kTileWords * 4;
    return bytes <= 0x7fffffffu;
}

int create_matrix(int device, const uint32_t* words, size_t n_words, int rows, int cols,
                  int row_words, float scale, loom_amd_matrix** out) {
    if (out == nullptr) return fail("out is null");
    *out = nullptr;
    if (words == nullptr) return fail("words is null");
    if (rows <= 0 || cols <= 0) return fail("rows and cols must be positive");
    if (row_words <= 0) row_words = ceil_div(cols, 16);
    if (row_words < ceil_div(cols, 16)) return fail("row_words < ceil(cols/16)");
    if (n_words < (size_t)rows * (size_t)row_words) {
        return fail("word count " + std::to_string(n_words) + " < rows*row_words " +
                    std::to_string((size_t)rows * (size_t)row_words));
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
        return fail("device " + std::to_string(device) + " is not visible");
    }
    if (!is_gfx950(device)) return fail("device is not gfx950");
    if (!tiles_fit(rows, cols)) return fail("matrix tiles exceed 2 GiB (the kernels use 32-bit buffer offsets)");
    DeviceGuard guard(device);
    auto* w = new loom_amd_matrix();
    Matrix& m = w->m;
    m.rows = rows;
    m.cols = cols;
    m.ntiles = ceil_div(rows, kTileRows);
    m.ktiles = ceil_div(cols, kTileCols);
    m.scale = scale;
    m.device = device;
    uint32_t* staging = nullptr;
    const size_t src_bytes = (size_t)rows * (size_t)row_words * 4;
    hipError_t e = hipMalloc(&staging, src_bytes);
    if (e == hipSuccess) e = gemm_prepare(device);
    if (e == hipSuccess) e = hipMalloc(&m.tiles, m.bytes());
    if (e == hipSuccess) e = hipMemcpy(staging, words, src_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_repack(staging, rows, cols, row_words, &m, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (staging) (void)hipFree(staging);
    if (e != hipSuccess) {
        if (m.tiles) (void)hipFree(m.tiles);
        delete w;
        return fail_hip("matrix upload", e);
    }
    *out = w;
    return 0;
}

int create_matrix_ms_offline(int device, const uint8_t* packed, int rows, int cols, float scale,
                             loom_amd_matrix** out) {
    if (out == nullptr) return fail("out is null");
    *out = nullptr;
    if (packed == nullptr) return fail("packed bytes are null");
    if (rows <= 0 || cols <= 0) return fail("rows and cols must be positive");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
        return fail("device " + std::to_string(device) + " is not visible");
    }
    if (!is_gfx950(device)) return fail("device is not gfx950");
    if (!tiles_fit(rows, cols)) return fail("matrix tiles exceed 2 GiB (the kernels use 32-bit buffer offsets)");
    DeviceGuard guard(device);
    auto* w = new loom_amd_matrix();
    Matrix& m = w->m;
    m.rows = rows;
    m.cols = cols;
    m.ntiles = ceil_div(rows, kTileRows);
    m.ktiles = ceil_div(cols, kTileCols);
    m.scale = scale;
    m.device = device;
    const int row_words = ceil_div(cols, 16);
    const size_t packed_bytes = (size_t)(rows / 4) * cols;
    uint8_t* dpacked = nullptr;
    uint32_t* staging = nullptr;
    hipError_t e = hipMalloc(&dpacked, packed_bytes ? packed_bytes : 1);
    if (e == hipSuccess) e = hipMalloc(&staging, (size_t)rows * row_words * 4);
    if (e == hipSuccess) e = gemm_prepare(device);
    if (e == hipSuccess) e = hipMalloc(&m.tiles, m.bytes());
    if (e == hipSuccess && packed_bytes) e = hipMemcpy(dpacked, packed, packed_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_ms_offline_to_words(dpacked, rows, cols, staging, nullptr);
    if (e == hipSuccess) e = launch_repack(staging, rows, cols, row_words, &m, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (staging) (void)hipFree(staging);
    if (dpacked) (void)hipFree(dpacked);
    if (e != hipSuccess) {
        if (m.tiles) (void)hipFree(m.tiles);
        delete w;
        return fail_hip("offline matrix upload", e);
    }
    *out = w;
    return 0;
}

namespace {

const char* const kTuneNames[] = {
    "LOOM_AMD_GEMM_TILE",   "LOOM_AMD_GEMM_SPLIT",   "LOOM_AMD_GEMM_GROUP",   "LOOM_AMD_SMALLM",
    "LOOM_AMD_SKINNY_NT",   "LOOM_AMD_SKINNY_NTR",   "LOOM_AMD_FUSED_NTR",    "LOOM_AMD_FUSED_WAVES",
    "LOOM_AMD_GEMV_STREAM", "LOOM_AMD_STREAM_WAVES", "LOOM_AMD_STREAM_DEPTH", "LOOM_AMD_ATTN_QT",
    "LOOM_AMD_UNFUSED_ROPE", "LOOM_AMD_UNFUSED_NORM", "LOOM_AMD_GEMM_NJ", "LOOM_AMD_ROWNORM_WAVE",
    "LOOM_AMD_QUANT_GROUPS", "LOOM_AMD_LM_SCREEN"};
constexpr int kTuneCount = (int)(sizeof(kTuneNames) / sizeof(kTuneNames[0]));

struct TuneSnapshot {
    bool set[kTuneCount];
    int value[kTuneCount];
};

std::mutex g_tune_mu;
std::atomic<const TuneSnapshot*> g_tune{nullptr};
std::vector<std::unique_ptr<TuneSnapshot>> g_tune_all;  // every snapshot lives until exit

const TuneSnapshot* read_tuning_locked() {
    auto t = std::make_unique<TuneSnapshot>();
    for (int i = 0; i < kTuneCount; ++i) {
        const char* v = getenv(kTuneNames[i]);
        t->set[i] = v && *v;
        t->value[i] = t->set[i] ? atoi(v) : 0;
    }
    g_tune_all.push_back(std::move(t));
    return g_tune_all.back().get();
}

}  // namespace

int tune_int(const char* name, int dflt) {
    const TuneSnapshot* t = g_tune.load(std::memory_order_acquire);
    if (!t) {
        std::lock_guard<std::mutex> lock(g_tune_mu);
        t = g_tune.load(std::memory_order_acquire);
        if (!t) {
            t = read_tuning_locked();
            g_tune.store(t, std::memory_order_release);
        }
    }
    for (int i = 0; i < kTuneCount; ++i) {
        if (strcmp(name, kTuneNames[i]) == 0) return t->set[i] ? t->value[i] : dflt;
    }
    return dflt;
}

void reload_tuning() {
    std::lock_guard<std::mutex> lock(g_tune_mu);
    g_tune.store(read_tuning_locked(), std::memory_order_release);
}

}  // namespace lamd

using namespace lamd;

extern "C" {

int loom_amd_matrix_from_ms_offline(int device, const uint8_t* packed, int rows, int cols,
                                    float scale, loom_amd_matrix** out) {
    return create_matrix_ms_offline(device, packed, rows, cols, scale, out);
}

// bitNetQuantValue (poly/bitnet_cpu.go:134-146): an fp32 division, rounded
// half away from zero in fp64, clamped to [-1, 1]; Go's int(float64) on amd64
// turns NaN and out-of-range values into INT64_MIN, hence -1.  Returns loom's
// storage code (poly/bitnet_cpu.go:498-507): -1 -> 0, 0 -> 1, 1 -> 2.
static uint32_t quant_code(float v, float scale) {
    if (scale == 0.0f) scale = 1.0f;
    const double r = round((double)(v / scale));
    long long q;
    if (!(r >= -9223372036854775808.0 && r < 9223372036854775808.0)) {
        q = INT64_MIN;
    } else {
        q = (long long)r;
    }
    if (q > 1) q = 1;
    if (q < -1) q = -1;
    return (uint32_t)(q + 1);
}

// packFloat32AsBitNetTernaryMatrix (poly/bitnet_cpu.go:934-977) into loom's
// row-major words (16 codes per u32, column c at bits 2*(c%16)).  The absmean
// scale (poly/bitnet_cpu.go:119-132) is one sequential fp64 sum; the per-weight
// codes are independent and are formed on several host threads.
float pack_float32_words(const float* w, int rows, int cols, std::vector<uint32_t>* words) {
    const size_t total = (size_t)rows * (size_t)cols;
    double sum_abs = 0.0;
    bool already = true;
    for (size_t i = 0; i < total; ++i) {
        const float v = w[i];
        sum_abs += fabs((double)v);
        if (!(fabs((double)v) < 1e-6 || fabs((double)(v - 1.0f)) < 1e-6 ||
              fabs((double)(v + 1.0f)) < 1e-6)) {
            already = false;
        }
    }
    float scale = (float)(sum_abs / (double)total);
    if (scale == 0.0f) scale = 1.0f;
    if (already) scale = 1.0f;
    const int rw = ceil_div(cols, 16);
    words->assign((size_t)rows * rw, 0u);
    uint32_t* out = words->data();
    const unsigned hw = std::thread::hardware_concurrency();
    const int nt = (int)std::max(1u, std::min(hw ? hw : 1u, 16u));
    auto work = [&](int r0, int r1) {
        for (int r = r0; r < r1; ++r) {
            const float* src = w + (size_t)r * cols;
            uint32_t* dst = out + (size_t)r * rw;
            for (int c = 0; c < cols; ++c) dst[c / 16] |= quant_code(src[c], scale) << (2 * (c % 16));
        }
    };
    if (nt <= 1 || total < ((size_t)1 << 20)) {
        work(0, rows);
    } else {
        std::vector<std::thread> pool;
        const int per = ceil_div(rows, nt);
        for (int t = 0; t < nt; ++t) {
            const int r0 = t * per, r1 = std::min(rows, r0 + per);
            if (r0 < r1) pool.emplace_back(work, r0, r1);
        }
        for (auto& th : pool) th.join();
    }
    return scale;
}

int loom_amd_matrix_from_float32(int device, const float* master, int rows, int cols,
                                 loom_amd_matrix** out, float* scale_out) {
    if (out) *out = nullptr;
    if (master == nullptr) return fail("master is null");
    if (rows <= 0 || cols <= 0) return fail("rows and cols must be positive");
    std::vector<uint32_t> words;
    const float scale = pack_float32_words(master, rows, cols, &words);
    if (scale_out) *scale_out = scale;
    return create_matrix(device, words.data(), words.size(), rows, cols, ceil_div(cols, 16), scale, out);
}

const char* loom_amd_last_error(void) { return g_amd_error.c_str(); }

int loom_amd_device_count(void) { return visible_gfx950(); }

const char* loom_amd_kernel_variant(int m) { return kernel_variant(m); }

int loom_amd_matrix_create(int device, const uint32_t* words, size_t n_words, int rows,
                           int cols, int row_words, float scale, loom_amd_matrix** out) {
    return create_matrix(device, words, n_words, rows, cols, row_words, scale, out);
}

static uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}

// decodeEntityBitNetTernaryBlob (poly/entity_bitnet.go:57-88).
int loom_amd_matrix_from_entity_blob(int device, const void* blob, size_t len,
                                     loom_amd_matrix** out, size_t* consumed) {
    if (out) *out = nullptr;
    if (blob == nullptr) return fail("blob is null");
    const uint8_t* raw = (const uint8_t*)blob;
    if (len < 24) return fail("bitnet ternary blob too short");
    const int rows = (int)rd32(raw + 0);
    const int cols = (int)rd32(raw + 4);
    uint32_t sbits = rd32(raw + 12);
    float scale;
    memcpy(&scale, &sbits, 4);
    int row_words = (int)rd32(raw + 16);
    const uint32_t n_words = rd32(raw + 20);
    const size_t need = 24 + (size_t)n_words * 4;
    if (len < need) {
        return fail("bitnet ternary blob truncated: have " + std::to_string(len) + " need " +
                    std::to_string(need));
    }
    if (row_words <= 0) row_words = ceil_div(cols, 16);
    std::vector<uint32_t> words(n_words);
    if (n_words) memcpy(words.data(), raw + 24, (size_t)n_words * 4);  // little-endian host
    if (consumed) *consumed = need;
    return create_matrix(device, words.data(), n_words, rows, cols, row_words, scale, out);
}

void loom_amd_matrix_release(loom_amd_matrix* w) {
    if (w == nullptr) return;
    if (w->m.tiles) {
        DeviceGuard guard(w->m.device);
        (void)hipFree(w->m.tiles);
    }
    delete w;
}

int loom_amd_matrix_shape(const loom_amd_matrix* w, int* rows, int* cols, float* scale,
                          size_t* device_bytes) {
    if (check_matrix(w, "w")) return -1;
    if (rows) *rows = w->m.rows;
    if (cols) *cols = w->m.cols;
    if (scale) *scale = w->m.scale;
    if (device_bytes) *device_bytes = w->m.bytes();
    return 0;
}

const void* loom_amd_matrix_tiles(const loom_amd_matrix* w) {
    return w ? (const void*)w->m.tiles : nullptr;
}

static int check_ldq(int k, int ldq) {
    if (ldq < k || ldq % kTileCols != 0) {
        return fail("ldq must be >= k and a multiple of 256");
    }
    return 0;
}

int loom_amd_quantize_rows(const float* x, int m, int k, int8_t* xq, int ldq, float* amax,
                           int32_t* xsum, void* stream) {
    if (m < 0 || k <= 0) return fail("bad shape");
    if (m == 0) return 0;
    if (!x || !xq || !amax || !xsum) return fail("null buffer");
    if (check_ldq(k, ldq)) return -1;
    hipError_t e = launch_act_quant(x, k, m, k, xq, ldq, amax, xsum, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail_hip("quantize_rows", e);
}

int loom_amd_quantize_rows_f64(const double* x, int m, int k, int8_t* xq, int ldq,
                               float* amax, int32_t* xsum, void* stream) {
    if (m < 0 || k <= 0) return fail("bad shape");
    if (m == 0) return 0;
    if (!x || !xq || !amax || !xsum) return fail("null buffer");
    if (check_ldq(k, ldq)) return -1;
    hipError_t e = launch_act_quant_f64(x, k, m, k, xq, ldq, amax, xsum, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail_hip("quantize_rows_f64", e);
}

int loom_amd_ternary_matmul(const loom_amd_matrix* w, const int8_t* xq, int ldq,
                            const float* amax, const int32_t* xsum, int m, float* out,
                            int32_t* acc, void* stream) {
    if (check_matrix(w, "w")) return -1;
    if (m < 0) return fail("bad shape");
    if (m == 0) return 0;
    if (!xq || !amax || !xsum || !out) return fail("null buffer");
    if (ldq < w->m.ktiles * kTileCols || ldq % kTileCols != 0) {
        return fail("ldq must be a multiple of 256 covering the padded columns");
    }
    if (((uintptr_t)xq & 15) != 0) return fail("xq must be 16-byte aligned");
    DeviceGuard guard(w->m.device);
    QuantAct a{xq, ldq, amax, xsum};
    Epilogue epi;
    epi.kind = EPI_DENSE;
    epi.out = out;
    epi.ldo = w->m.rows;
    epi.acc0 = acc;
    hipError_t e = launch_matmul(&w->m, nullptr, a, m, epi, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail_hip("ternary_matmul", e);
}

int loom_amd_norm_quant_rows(float* h, int m, int n, const float* weight, double eps,
                             int norm_mode, int8_t* hq, int ldq, float* amax, int32_t* xsum,
                             void* stream) {
    if (m < 0 || n <= 0) return fail("bad shape");
    if (m == 0) return 0;
    if (!h || !hq || !amax || !xsum) return fail("null buffer");
    if (check_ldq(n, ldq)) return -1;
    if (((uintptr_t)hq & 15) != 0) return fail("hq must be 16-byte aligned");
    if (n > kMaxNormCols || (norm_mode == LOOM_AMD_NORM_STRICT && n > kMaxStrictNormCols)) {
        return fail("norm rows are limited to 8192 values (strict: 8064)");
    }
    hipError_t e = launch_norm_quant(h, n, m, n, weight, eps, norm_mode == LOOM_AMD_NORM_STRICT,
                                     hq, ldq, amax, xsum, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail_hip("norm_quant_rows", e);
}

int loom_amd_ordered_sum_rows(const double* terms, int m, int n, double s0, double* out,
                              int threads, void* stream) {
    if (m < 0 || n <= 0) return fail("bad shape");
    if (m == 0) return 0;
    if (!terms || !out) return fail("null buffer");
    if (n > kMaxStrictNormCols) return fail("ordered sums are limited to 8064 terms per row");
    if (threads != 64 && threads != 256 && threads != 512) return fail("threads must be 64, 256 or 512");
    hipError_t e = launch_ordered_sum_rows(terms, m, n, s0, out, threads, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail_hip("ordered_sum_rows", e);
}

int loom_amd_reload_tuning(void) {
    reload_tuning();
    return 0;
}

int loom_amd_exp_rows(const double* x, long n, double* y, void* stream) {
    if (n < 0) return fail("bad size");
    if (n == 0) return 0;
    if (!x || !y) return fail("null buffer");
    hipError_t e = launch_exp_rows(x, n, y, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail_hip("exp_rows", e);
}

int loom_amd_dense_forward(const loom_amd_matrix* w, const float* x, int m, int activation,
                           float* pre, float* post, const float* residual,
                           const loom_amd_dense_taps* taps, void* stream) {
    if (check_matrix(w, "w")) return -1;
    if (m < 0) return fail("bad shape");
    if (m == 0) return 0;
    if (!x || !pre) return fail("null buffer");
    const Matrix& W = w->m;
    DeviceGuard guard(W.device);
    hipStream_t s = (hipStream_t)stream;
    Epilogue epi;
    epi.kind = EPI_DENSE;
    epi.activation = activation;
    epi.residual = residual;
    epi.out = pre;
    epi.post = post;
    epi.ldo = W.rows;
    epi.acc0 = taps ? taps->acc : nullptr;
    if (fused_quant_ok(m, W.cols, x)) {
        // decode-sized batches: quantization runs inside the matmul launch
        hipError_t e = launch_matmul_fused(&W, nullptr, x, m, epi, taps ? taps->xq : nullptr,
                                           taps ? taps->amax : nullptr, s);
        return e == hipSuccess ? 0 : fail_hip("dense_forward fused", e);
    }
    const int ldq = ld_for(W.cols);
    Layout L;
    const size_t o_xq = L.take((size_t)m * ldq);
    const size_t o_am = L.take((size_t)m * 4);
    const size_t o_xs = L.take((size_t)m * 4);
    std::string err;
    char* base = (char*)scratch(W.device, L.off, &err);
    if (!base) return fail(err);
    int8_t* xq = (int8_t*)(base + o_xq);
    float* am = (float*)(base + o_am);
    int32_t* xs = (int32_t*)(base + o_xs);
    hipError_t e = launch_act_quant(x, W.cols, m, W.cols, xq, ldq, am, xs, s);
    if (e != hipSuccess) return fail_hip("dense_forward quantize", e);
    QuantAct a{xq, ldq, am, xs};
    e = launch_matmul(&W, nullptr, a, m, epi, s);
    if (e != hipSuccess) return fail_hip("dense_forward matmul", e);
    if (taps && taps->xq) {
        e = hipMemcpy2DAsync(taps->xq, W.cols, xq, ldq, W.cols, m, hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return fail_hip("dense_forward tap xq", e);
    }
    if (taps && taps->amax) {
        e = hipMemcpyAsync(taps->amax, am, (size_t)m * 4, hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return fail_hip("dense_forward tap amax", e);
    }
    return 0;
}

int loom_amd_swiglu_forward(const loom_amd_matrix* gate, const loom_amd_matrix* up,
                            const loom_amd_matrix* down, const float* bias,
                            const float* inner_norm, double eps, int activation,
                            int norm_mode, const float* x, int m, float* out,
                            const float* residual, float* h_out,
                            const loom_amd_swiglu_taps* taps, void* stream) {
    if (check_matrix(gate, "gate") || check_matrix(up, "up") || check_matrix(down, "down")) {
        return -1;
    }
    const Matrix& G = gate->m;
    const Matrix& U = up->m;
    const Matrix& D = down->m;
    const int hidden = G.cols, inter = G.rows;
    if (U.rows != inter || U.cols != hidden || D.rows != hidden || D.cols != inter) {
        return fail("swiglu shapes disagree: gate/up must be inter x hidden, down hidden x inter");
    }
    if (G.device != U.device || G.device != D.device) return fail("matrices on different devices");
    if (m < 0) return fail("bad shape");
    if (m == 0) return 0;
    if (!x || !out) return fail("null buffer");
    const int strict = norm_mode == LOOM_AMD_NORM_STRICT;
    if (inter > kMaxNormCols || (strict && inter > kMaxStrictNormCols)) {
        return fail("swiglu intermediate width is limited to 8192 (strict norm: 8064)");
    }
    DeviceGuard guard(G.device);
    // a decode row: the down projection's workgroups normalize and quantize
    // h themselves (as the decoder block does), reading the gate product from
    // scratch and writing the normalized rows to h_out; LOOM_AMD_UNFUSED_NORM=1
    // keeps the separate norm launch, which normalizes h in place
    const bool fuse_down = tune_int("LOOM_AMD_UNFUSED_NORM", 0) != 1 && norm_fused_ok(m, inter, strict, true) &&
                           ((uintptr_t)inner_norm & 15) == 0 && ((uintptr_t)h_out & 15) == 0;
    const int ldx = ld_for(hidden), ldh = ld_for(inter);
    Layout L;
    const size_t o_xq = L.take((size_t)m * ldx);
    const size_t o_am = L.take((size_t)m * 4);
    const size_t o_xs = L.take((size_t)m * 4);
    const size_t o_h = L.take(h_out && !fuse_down ? 0 : (size_t)m * inter * 4);
    const size_t o_hq = L.take((size_t)m * ldh);
    const size_t o_ham = L.take((size_t)m * 4);
    const size_t o_hs = L.take((size_t)m * 4);
    std::string err;
    char* base = (char*)scratch(G.device, L.off, &err);
    if (!base) return fail(err);
    int8_t* xq = (int8_t*)(base + o_xq);
    float* am = (float*)(base + o_am);
    int32_t* xs = (int32_t*)(base + o_xs);
    float* h = h_out && !fuse_down ? h_out : (float*)(base + o_h);
    int8_t* hq = (int8_t*)(base + o_hq);
    float* ham = (float*)(base + o_ham);
    int32_t* hs = (int32_t*)(base + o_hs);
    hipStream_t s = (hipStream_t)stream;

    Epilogue gu;
    gu.kind = EPI_SWIGLU;
    gu.activation = activation;
    gu.bias0 = bias ? bias : nullptr;
    gu.bias1 = bias ? bias + inter : nullptr;
    gu.out = h;
    gu.ldo = inter;
    gu.acc0 = taps ? taps->acc_gate : nullptr;
    gu.acc1 = taps ? taps->acc_up : nullptr;
    const bool fused = fused_quant_ok(m, hidden, x);
    hipError_t e;
    if (fused) {
        e = launch_matmul_fused(&G, &U, x, m, gu, taps ? taps->xq : nullptr,
                                taps ? taps->amax : nullptr, s);
    } else {
        e = launch_act_quant(x, hidden, m, hidden, xq, ldx, am, xs, s);
        if (e != hipSuccess) return fail_hip("swiglu quantize", e);
        QuantAct a{xq, ldx, am, xs};
        e = launch_matmul(&G, &U, a, m, gu, s);
    }
    if (e != hipSuccess) return fail_hip("swiglu gate/up", e);
    Epilogue dn;
    dn.kind = EPI_DENSE;
    dn.activation = -1;
    dn.bias0 = bias ? bias + 2 * inter : nullptr;
    dn.residual = residual;
    dn.out = out;
    dn.ldo = hidden;
    dn.acc0 = taps ? taps->acc_down : nullptr;
    if (fuse_down) {
        NormTaps nt;
        nt.rows = h_out;
        nt.xq = taps ? taps->hq : nullptr;
        nt.amax = taps ? taps->hamax : nullptr;
        e = launch_matmul_norm(&D, nullptr, h, nullptr, m, NORM_INNER_F32, strict, inner_norm,
                               eps <= 0.0 ? 1e-5 : eps, dn, nullptr, s, &nt);  // (launch_norm_quant's default eps)
        if (e != hipSuccess) return fail_hip("swiglu inner norm + down", e);
    } else {
        e = launch_norm_quant(h, inter, m, inter, inner_norm, eps, strict, hq, ldh, ham, hs, s);
        if (e != hipSuccess) return fail_hip("swiglu inner norm", e);
        QuantAct b{hq, ldh, ham, hs};
        e = launch_matmul(&D, nullptr, b, m, dn, s);
        if (e != hipSuccess) return fail_hip("swiglu down", e);
    }
    if (taps) {
        if (!fused && taps->xq) e = hipMemcpy2DAsync(taps->xq, hidden, xq, ldx, hidden, m, hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess && !fused && taps->amax) e = hipMemcpyAsync(taps->amax, am, (size_t)m * 4, hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess && !fuse_down && taps->hq)
            e = hipMemcpy2DAsync(taps->hq, inter, hq, ldh, inter, m, hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess && !fuse_down && taps->hamax)
            e = hipMemcpyAsync(taps->hamax, ham, (size_t)m * 4, hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return fail_hip("swiglu taps", e);
    }
    return 0;
}

}  // extern "C"
