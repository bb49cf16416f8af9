// noalloc.hip -- loom_amd_dense_forward_noalloc: the Dense forward of
// loom_amd_dense_forward for callers that must not allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  It has no counterpart in loom.
//
// Where loom_amd_dense_forward stages the quantized rows (int8 rows, amax,
// sum(xq)) of token rows the matmul launch does not quantize itself (more
// than four, or than eight for K <= 4096) in the per-device scratch arena,
// which grows with hipMalloc, this entry point stages them in `scratch`, a
// fixed device array of kNoAllocScratchBytes that every GPU the library runs
// on holds until the process ends.  Its device address is looked up once per
// device (hipGetSymbolAddress, on the first call there) and kept; host code
// passes only that address to kernels.  The GEMM's split-K workspace is
// allocated when a matrix is created, never by a call, so the call allocates
// nothing.  Every call on one GPU shares its array: calls that overlap on one
// GPU (two host threads, or two streams) race and must be serialized by the
// caller.  Nothing in the array needs to start at zero: the quantization
// kernel writes every byte the matmul reads (including the zero padding
// past K).
#include "api_util.hpp"
#include "lamd.hpp"
#include "loom_accel_amd.h"

#include <mutex>
#include <string>
#include <vector>

namespace {

constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;  // 8 MiB per GPU

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_ptr_mu;
std::vector<void*> g_ptr;  // device address of `scratch`, per device (null until looked up)

// Address of the calling device's copy of `scratch`; looked up on the first
// call on each device, with that device current.
void* scratch_ptr(int device, std::string* err) {
    std::lock_guard<std::mutex> lock(g_ptr_mu);
    if ((int)g_ptr.size() <= device) g_ptr.resize(device + 1, nullptr);
    if (g_ptr[device]) return g_ptr[device];
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
        *err = std::string("dense_forward_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e);
        return nullptr;
    }
    g_ptr[device] = p;
    return p;
}

}  // namespace

using namespace lamd;

extern "C" {

int loom_amd_dense_forward_noalloc(const loom_amd_matrix* w, const float* x, int m, int activation,
                                   float* pre, float* post, const float* residual, void* stream) {
    if (w == nullptr || w->m.tiles == nullptr) return fail("w matrix is null");
    if (m < 0) return fail("bad shape");
    if (m == 0) return 0;
    if (!x || !pre) return fail("null buffer");
    const Matrix& W = w->m;
    const int ldq = pad_cols(W.cols);
    Layout L;
    const size_t o_xq = L.take((size_t)m * ldq);
    const size_t o_am = L.take((size_t)m * 4);
    const size_t o_xs = L.take((size_t)m * 4);
    if (L.off > kNoAllocScratchBytes) {
        return fail("dense_forward_noalloc: " + std::to_string(m) + " rows of " +
                    std::to_string(W.cols) + " columns need " + std::to_string(L.off) +
                    " bytes of quantized rows, more than the fixed " +
                    std::to_string(kNoAllocScratchBytes) + " bytes (use loom_amd_dense_forward)");
    }
    DeviceGuard guard(W.device);
    hipStream_t s = (hipStream_t)stream;
    Epilogue epi;
    epi.kind = EPI_DENSE;
    epi.activation = activation;
    epi.residual = residual;
    epi.out = pre;
    epi.post = post;
    epi.ldo = W.rows;
    if (fused_quant_ok(m, W.cols, x)) {
        // decode-sized batches quantize inside the matmul launch: no staging
        hipError_t e = launch_matmul_fused(&W, nullptr, x, m, epi, nullptr, nullptr, s);
        return e == hipSuccess ? 0 : fail_hip("dense_forward_noalloc fused", e);
    }
    std::string err;
    char* base = (char*)scratch_ptr(W.device, &err);
    if (!base) return fail(err);
    int8_t* xq = (int8_t*)(base + o_xq);
    float* am = (float*)(base + o_am);
    int32_t* xs = (int32_t*)(base + o_xs);
    hipError_t e = launch_act_quant(x, W.cols, m, W.cols, xq, ldq, am, xs, s);
    if (e != hipSuccess) return fail_hip("dense_forward_noalloc quantize", e);
    QuantAct a{xq, ldq, am, xs};
    e = launch_matmul(&W, nullptr, a, m, epi, s);
    return e == hipSuccess ? 0 : fail_hip("dense_forward_noalloc matmul", e);
}

}  // extern "C"
