// plugin.hip -- loom's v2 vendor plugin ABI (include/loom_accel.h) for gfx950.
//
// Layers:
//   "BitNetLinear"  one ternary Dense layer, DenseForwardPackedTernaryCPU
//                   (poly/dense.go:66-101); weights: one BITNET_TERNARY blob.
//   "BitNetSwiGLU"  one ternary SwiGLU FFN, SwiGLUForwardPackedTernaryCPU
//                   (poly/swiglu.go:270-322); weights: gate, up, down blobs,
//                   then optionally n fp32 inner-norm weights, then (with
//                   bias=1) the 2n + k fp32 biases [gate | up | down] of the
//                   layer's Master tail (poly/swiglu.go:276-281).
// dtype "TERNARY"; size_label
// "m=..,k=..,n=..[,act=..][,eps=..][,norm=strict|fast][,bias=0|1]".
// Only device "GPU" exists: loom's own CPU path is the CPU implementation.
#include "api_util.hpp"
#include "lamd.hpp"
#include "loom_accel.h"
#include "loom_accel_amd.h"

#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <mutex>
#include <string>

struct loom_accel_plugin {
    int device = 0;
    std::string last_error;
    std::mutex mu;
};

struct loom_accel_compiled_layer {
    int kind = 0;  // 0 BitNetLinear, 1 BitNetSwiGLU
    int m = 0, k = 0, n = 0;
    int activation = -1;
    double eps = 1e-5;
    int norm_mode = LOOM_AMD_NORM_STRICT;
    int device = 0;
    loom_amd_matrix* w[3] = {nullptr, nullptr, nullptr};
    float* d_norm = nullptr;
    float* d_bias = nullptr;
    float* d_in = nullptr;
    float* d_out = nullptr;
    // pinned staging of the caller's host buffers: copies between pageable
    // memory and the device need not have finished when they are queued
    void* h_in = nullptr;
    void* h_out = nullptr;
    hipStream_t stream = nullptr;
    size_t in_bytes = 0, out_bytes = 0;
};

namespace {

using Clock = std::chrono::steady_clock;

thread_local std::string g_open_error;

void set_err(char* err, size_t err_len, const std::string& msg) {
    if (err == nullptr || err_len == 0) return;
    size_t n = msg.size() < err_len - 1 ? msg.size() : err_len - 1;
    memcpy(err, msg.data(), n);
    err[n] = '\0';
}

double ms_since(Clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

struct Spec {
    int kind = -1;
    int m = 0, k = 0, n = 0;
    int activation = -1;
    double eps = 1e-5;
    int norm_mode = LOOM_AMD_NORM_STRICT;
    int bias = 0;
};

bool parse_int(const std::string& v, int* out) {
    if (v.empty()) return false;
    char* end = nullptr;
    long x = strtol(v.c_str(), &end, 10);
    if (*end != '\0' || x < -(1L << 30) || x > (1L << 30)) return false;
    *out = (int)x;
    return true;
}

// Parses the desc into a Spec; returns false with a message on any mismatch.
bool parse_desc(const loom_accel_layer_desc* desc, Spec* s, std::string* why) {
    if (desc == nullptr) {
        *why = "desc is null";
        return false;
    }
    const std::string name = desc->layer_name ? desc->layer_name : "";
    const std::string dtype = desc->dtype ? desc->dtype : "";
    if (name == "BitNetLinear") {
        s->kind = 0;
    } else if (name == "BitNetSwiGLU") {
        s->kind = 1;
        s->activation = 1;
    } else {
        *why = "unknown layer: " + name + " (expected BitNetLinear or BitNetSwiGLU)";
        return false;
    }
    if (dtype != "TERNARY") {
        *why = "unknown dtype: " + dtype + " (expected TERNARY)";
        return false;
    }
    const std::string label = desc->size_label ? desc->size_label : "";
    size_t pos = 0;
    bool have_m = false, have_k = false, have_n = false;
    while (pos <= label.size()) {
        size_t comma = label.find(',', pos);
        if (comma == std::string::npos) comma = label.size();
        const std::string item = label.substr(pos, comma - pos);
        pos = comma + 1;
        if (item.empty()) continue;
        const size_t eq = item.find('=');
        if (eq == std::string::npos) {
            *why = "size label item without '=': " + item;
            return false;
        }
        const std::string key = item.substr(0, eq), val = item.substr(eq + 1);
        bool ok = true;
        if (key == "m") {
            ok = parse_int(val, &s->m) && s->m > 0;
            have_m = true;
        } else if (key == "k") {
            ok = parse_int(val, &s->k) && s->k > 0;
            have_k = true;
        } else if (key == "n") {
            ok = parse_int(val, &s->n) && s->n > 0;
            have_n = true;
        } else if (key == "act") {
            ok = parse_int(val, &s->activation) && s->activation >= -1 && s->activation <= 6;
        } else if (key == "bias") {
            ok = s->kind == 1 && (val == "0" || val == "1");
            s->bias = val == "1";
        } else if (key == "eps") {
            char* end = nullptr;
            s->eps = strtod(val.c_str(), &end);
            ok = !val.empty() && *end == '\0';
        } else if (key == "norm") {
            if (val == "strict") {
                s->norm_mode = LOOM_AMD_NORM_STRICT;
            } else if (val == "fast") {
                s->norm_mode = LOOM_AMD_NORM_FAST;
            } else {
                ok = false;
            }
        } else {
            ok = false;
        }
        if (!ok) {
            *why = "bad size label item: " + item;
            return false;
        }
    }
    if (!have_m || !have_k || !have_n) {
        *why = "size label must carry m, k and n: '" + label + "'";
        return false;
    }
    return true;
}

size_t blob_bytes(int rows, int cols) {
    return 24 + (size_t)rows * (size_t)((cols + 15) / 16) * 4;
}

size_t spec_bias_bytes(const Spec& s) {
    return s.kind == 1 && s.bias ? (size_t)(2 * s.n + s.k) * 4 : 0;
}

size_t spec_weight_bytes(const Spec& s) {
    if (s.kind == 0) return blob_bytes(s.n, s.k);
    return 2 * blob_bytes(s.n, s.k) + blob_bytes(s.k, s.n) + (size_t)s.n * 4 + spec_bias_bytes(s);
}

int read_blob_shape(const uint8_t* p, size_t len, int* rows, int* cols) {
    if (len < 24) return -1;
    *rows = (int)(p[0] | p[1] << 8 | p[2] << 16 | (uint32_t)p[3] << 24);
    *cols = (int)(p[4] | p[5] << 8 | p[6] << 16 | (uint32_t)p[7] << 24);
    return 0;
}

void release(loom_accel_compiled_layer* l) {
    if (l == nullptr) return;
    int prev = -1;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(l->device);
    for (auto*& w : l->w) {
        loom_amd_matrix_release(w);
        w = nullptr;
    }
    if (l->d_norm) (void)hipFree(l->d_norm);
    if (l->d_bias) (void)hipFree(l->d_bias);
    if (l->d_in) (void)hipFree(l->d_in);
    if (l->d_out) (void)hipFree(l->d_out);
    if (l->h_in) (void)hipHostFree(l->h_in);
    if (l->h_out) (void)hipHostFree(l->h_out);
    if (l->stream) (void)hipStreamDestroy(l->stream);
    if (prev >= 0) (void)hipSetDevice(prev);
    delete l;
}

// Runs the layer on l->d_in -> l->d_out and waits for it.  The caller holds
// the device's lock: every layer on a device shares its scratch arena and
// split-K workspace (loom's Go glue has no lock of its own, and goroutines
// may call infer on two compiled layers at once).
int run(loom_accel_compiled_layer* l, std::string* why) {
    int rc;
    if (l->kind == 0) {
        // DispatchAccelForward hands one tensor back as both pre and post
        // (poly/accel_intel.go:223-225); the plugin returns Activate(pre).  The
        // epilogue thread that writes pre writes post after it, so pointing
        // both at d_out leaves the post-activation value there.
        rc = loom_amd_dense_forward(l->w[0], l->d_in, l->m, l->activation, l->d_out,
                                    l->activation != -1 ? l->d_out : nullptr, nullptr, nullptr,
                                    l->stream);
    } else {
        rc = loom_amd_swiglu_forward(l->w[0], l->w[1], l->w[2], l->d_bias, l->d_norm, l->eps,
                                     l->activation, l->norm_mode, l->d_in, l->m, l->d_out,
                                     nullptr, nullptr, nullptr, l->stream);
    }
    if (rc != 0) {
        *why = loom_amd_last_error();
        return -1;
    }
    hipError_t e = hipStreamSynchronize(l->stream);
    if (e != hipSuccess) {
        *why = std::string("hipStreamSynchronize: ") + hipGetErrorString(e);
        return -1;
    }
    return 0;
}

}  // namespace

extern "C" {

int loom_accel_api_version(void) { return LOOM_ACCEL_API_VERSION; }

const char* loom_accel_vendor_id(void) { return "amd"; }

int loom_accel_npu_available(void) { return lamd::visible_gfx950() > 0 ? 1 : 0; }

loom_accel_plugin* loom_accel_plugin_open(const char* device) {
    if (device == nullptr) {
        g_open_error = "device is null";
        return nullptr;
    }
    const std::string dev(device);
    int index = 0;
    if (dev == "GPU") {
        index = 0;
    } else if (dev.rfind("GPU:", 0) == 0 && parse_int(dev.substr(4), &index) && index >= 0) {
    } else if (dev == "CPU") {
        g_open_error =
            "device CPU is not provided by the amd plugin: loom's own CPU path is the CPU "
            "implementation (expected GPU)";
        return nullptr;
    } else {
        g_open_error = "unknown device: " + dev + " (expected GPU or GPU:<index>)";
        return nullptr;
    }
    if (index >= lamd::visible_gfx950()) {
        g_open_error = "no gfx950 GPU device available at index " + std::to_string(index);
        return nullptr;
    }
    auto* p = new loom_accel_plugin();
    p->device = index;
    return p;
}

void loom_accel_plugin_close(loom_accel_plugin* plugin) { delete plugin; }

size_t loom_accel_weight_bytes(const loom_accel_layer_desc* desc) {
    Spec s;
    std::string why;
    if (!parse_desc(desc, &s, &why)) return 0;
    return spec_weight_bytes(s);
}

int loom_accel_compile_layer(loom_accel_plugin* plugin, const loom_accel_layer_desc* desc,
                             const void* weight_bytes, size_t weight_byte_len,
                             loom_accel_compiled_layer** out, double* compile_ms, char* err,
                             size_t err_len) {
    if (out == nullptr) {
        set_err(err, err_len, "out is null");
        return -1;
    }
    *out = nullptr;
    if (plugin == nullptr || desc == nullptr) {
        set_err(err, err_len, "plugin or desc is null");
        return -1;
    }
    auto fail = [&](const std::string& msg) {
        set_err(err, err_len, msg);
        std::lock_guard<std::mutex> lock(plugin->mu);
        plugin->last_error = msg;
        return -1;
    };
    Spec s;
    std::string why;
    if (!parse_desc(desc, &s, &why)) return fail(why);
    if (weight_bytes == nullptr) return fail("weight bytes are null");
    const size_t want = spec_weight_bytes(s);
    const size_t want_no_norm = s.kind == 1 ? want - (size_t)s.n * 4 : want;
    if (weight_byte_len != want && weight_byte_len != want_no_norm) {
        return fail("weight byte length " + std::to_string(weight_byte_len) + " != " +
                    std::to_string(want));
    }
    const auto t0 = Clock::now();
    auto* l = new loom_accel_compiled_layer();
    l->kind = s.kind;
    l->m = s.m;
    l->k = s.k;
    l->n = s.n;
    l->activation = s.activation;
    l->eps = s.eps;
    l->norm_mode = s.norm_mode;
    l->device = plugin->device;

    const uint8_t* p = (const uint8_t*)weight_bytes;
    size_t left = weight_byte_len;
    const int nmat = s.kind == 0 ? 1 : 3;
    for (int i = 0; i < nmat; ++i) {
        int rows = 0, cols = 0;
        const int want_rows = (s.kind == 1 && i == 2) ? s.k : s.n;
        const int want_cols = (s.kind == 1 && i == 2) ? s.n : s.k;
        if (read_blob_shape(p, left, &rows, &cols) != 0 || rows != want_rows ||
            cols != want_cols) {
            release(l);
            return fail("blob " + std::to_string(i) + " shape " + std::to_string(rows) + "x" +
                        std::to_string(cols) + " != " + std::to_string(want_rows) + "x" +
                        std::to_string(want_cols));
        }
        size_t used = 0;
        if (loom_amd_matrix_from_entity_blob(l->device, p, left, &l->w[i], &used) != 0) {
            std::string m = loom_amd_last_error();
            release(l);
            return fail(m);
        }
        p += used;
        left -= used;
    }
    int prev = -1;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(l->device);
    l->in_bytes = (size_t)s.m * s.k * 4;
    l->out_bytes = (size_t)s.m * (s.kind == 0 ? s.n : s.k) * 4;
    hipError_t e = hipStreamCreateWithFlags(&l->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&l->d_in, l->in_bytes);
    if (e == hipSuccess) e = hipMalloc(&l->d_out, l->out_bytes);
    if (e == hipSuccess) e = hipHostMalloc(&l->h_in, l->in_bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc(&l->h_out, l->out_bytes, hipHostMallocDefault);
    const size_t bias_bytes = spec_bias_bytes(s);
    if (e == hipSuccess && s.kind == 1 && left == (size_t)s.n * 4 + bias_bytes) {
        e = hipMalloc(&l->d_norm, (size_t)s.n * 4);
        if (e == hipSuccess) e = hipMemcpy(l->d_norm, p, (size_t)s.n * 4, hipMemcpyHostToDevice);
        p += (size_t)s.n * 4;
        left -= (size_t)s.n * 4;
    }
    if (e == hipSuccess && bias_bytes) {
        e = hipMalloc(&l->d_bias, bias_bytes);
        if (e == hipSuccess) e = hipMemcpy(l->d_bias, p, bias_bytes, hipMemcpyHostToDevice);
    }
    if (prev >= 0) (void)hipSetDevice(prev);
    if (e != hipSuccess) {
        release(l);
        return fail(std::string("compile: ") + hipGetErrorString(e));
    }
    *out = l;
    if (compile_ms) *compile_ms = ms_since(t0);
    return 0;
}

void loom_accel_release_layer(loom_accel_compiled_layer* layer) { release(layer); }

int loom_accel_layer_io_bytes(loom_accel_compiled_layer* layer, size_t* in_bytes,
                              size_t* out_bytes, char* err, size_t err_len) {
    if (layer == nullptr) {
        set_err(err, err_len, "invalid compiled layer");
        return -1;
    }
    if (in_bytes) *in_bytes = layer->in_bytes;
    if (out_bytes) *out_bytes = layer->out_bytes;
    return 0;
}

int loom_accel_first_infer(loom_accel_compiled_layer* layer, double* first_infer_ms, char* err,
                           size_t err_len) {
    if (layer == nullptr) {
        set_err(err, err_len, "invalid compiled layer");
        return -1;
    }
    const auto t0 = Clock::now();
    std::lock_guard<std::mutex> lock(lamd::device_mutex(layer->device));
    hipError_t e = hipMemsetAsync(layer->d_in, 0, layer->in_bytes, layer->stream);
    if (e != hipSuccess) {
        set_err(err, err_len, std::string("first_infer: ") + hipGetErrorString(e));
        return -1;
    }
    std::string why;
    if (run(layer, &why) != 0) {
        set_err(err, err_len, why);
        return -1;
    }
    if (first_infer_ms) *first_infer_ms = ms_since(t0);
    return 0;
}

int loom_accel_infer(loom_accel_compiled_layer* layer, const void* in, size_t in_bytes,
                     void* out, size_t out_bytes, double* infer_ms, char* err, size_t err_len) {
    if (layer == nullptr) {
        set_err(err, err_len, "invalid compiled layer");
        return -1;
    }
    if (in == nullptr || out == nullptr) {
        set_err(err, err_len, "in/out buffer is null");
        return -1;
    }
    if (in_bytes != layer->in_bytes) {
        set_err(err, err_len, "input byte size mismatch");
        return -1;
    }
    if (out_bytes != layer->out_bytes) {
        set_err(err, err_len, "output byte size mismatch");
        return -1;
    }
    const auto t0 = Clock::now();
    std::lock_guard<std::mutex> lock(lamd::device_mutex(layer->device));
    // run() leaves the stream idle, so the previous call's copies are done
    memcpy(layer->h_in, in, in_bytes);
    hipError_t e = hipMemcpyAsync(layer->d_in, layer->h_in, in_bytes, hipMemcpyHostToDevice,
                                  layer->stream);
    if (e != hipSuccess) {
        set_err(err, err_len, std::string("infer upload: ") + hipGetErrorString(e));
        return -1;
    }
    std::string why;
    if (run(layer, &why) != 0) {
        set_err(err, err_len, why);
        return -1;
    }
    e = hipMemcpyAsync(layer->h_out, layer->d_out, out_bytes, hipMemcpyDeviceToHost, layer->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(layer->stream);
    if (e != hipSuccess) {
        set_err(err, err_len, std::string("infer download: ") + hipGetErrorString(e));
        return -1;
    }
    memcpy(out, layer->h_out, out_bytes);
    if (infer_ms) *infer_ms = ms_since(t0);
    return 0;
}

const char* loom_accel_last_error(loom_accel_plugin* plugin) {
    if (plugin == nullptr) return g_open_error.c_str();
    std::lock_guard<std::mutex> lock(plugin->mu);
    return plugin->last_error.c_str();
}

}  // extern "C"
