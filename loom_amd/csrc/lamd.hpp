// lamd.hpp -- internal declarations of libloom_accel_amd.so (gfx950 only).
//
// Weight layout in HBM ("tile layout"), built once per matrix by repack_tiles:
//   * the matrix (rows = N outputs, cols = K inputs) is cut into tiles of
//     16 rows x 256 columns; rows pad to Np = 16*ceil(N/16), columns to
//     Kp = 256*ceil(K/256);
//   * tiles are stored row-tile major: tile (nt, kt) starts at word
//     (nt*ktiles + kt) * 256 and holds 64 lanes x 4 words (1 KiB), so one
//     wavefront reads a tile with one fully coalesced 128-bit load per lane;
//   * lane l of a tile owns weight row 16*nt + (l & 15) and columns
//     256*kt + 64*t + 16*(l >> 4) + c for word t (0..3), c (0..15): word t of
//     the 64 lanes covers the contiguous K step [64t, 64t+64) of the tile;
//   * inside a word, the 2-bit code of column c = 4*d + j sits at bit
//     8*j + 2*d, so (word >> 2*d) & 0x03030303 is four int8 codes for the
//     K-contiguous columns 4d..4d+3 -- one shift and one AND per dword, and
//     the four dwords of a word are exactly one MFMA 16x16x64 i8 operand.
//   Codes keep loom's meaning (0 -> -1, 1 -> 0, 2 -> +1, poly/bitnet_cpu.go:
//   498-507); the kernels multiply the raw codes and subtract sum(xq) per
//   token row, the identity loom's amd64 path uses (poly/bitnet_cpu.go:733-750).
//   Padding columns carry code 0 and meet zero activations.
//
// Activations: int8 rows of Kp bytes (zero padded), one fp32 amax and one
// int32 sum(xq) per row.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

namespace lamd {

constexpr int kTileRows = 16;
constexpr int kTileCols = 256;
constexpr int kTileWords = 256;  // 64 lanes x 4 u32
constexpr int kMaxNormCols = 8192;        // row width of the norm kernels (256 x 32 in registers)
constexpr int kMaxStrictNormCols = 8064;  // strict mode keeps n fp64 squares in 64 KB of LDS

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int pad_cols(int k) { return ceil_div(k, kTileCols) * kTileCols; }

// Device-resident repacked ternary matrix.
struct Matrix {
    int rows = 0;      // N (outputs)
    int cols = 0;      // K (inputs)
    int ntiles = 0;    // ceil(N/16)
    int ktiles = 0;    // ceil(K/256)
    float scale = 1.0f;
    uint32_t* tiles = nullptr;  // ntiles*ktiles*256 words (device)
    int device = 0;
    size_t bytes() const { return (size_t)ntiles * ktiles * kTileWords * 4; }
};

// Quantized activations for one matmul call (device pointers).
struct QuantAct {
    const int8_t* xq;    // rows x ldq
    int ldq;             // row stride in bytes (multiple of 256, >= Kp)
    const float* amax;   // per row
    const int32_t* xsum; // per row
};

// Epilogue selector of the matmul kernels.
enum EpiKind : int {
    EPI_DENSE = 0,   // pre = fp32(fp64(acc)*os) [+bias]; post = Activate(pre); [+residual]
    EPI_SWIGLU = 1,  // h = fp32(gateprod(fp64(acc_g)*os_g + bg, fp64(acc_u)*os_u + bu))
    EPI_ACC = 2,     // only the int32 accumulators (acc0, M x N); the caller rescales
};

struct Epilogue {
    int kind = EPI_DENSE;
    int activation = -1;       // loom ActivationType
    const float* bias0 = nullptr;  // dense bias or gate bias (length N)
    const float* bias1 = nullptr;  // up bias (length N)
    const float* residual = nullptr;  // M x N, added in fp32 after the cast
    float* out = nullptr;      // M x ldo (pre-activation / h)
    float* post = nullptr;     // M x ldo (post-activation), optional
    int ldo = 0;
    int32_t* acc0 = nullptr;   // M x N debug tap (acc of matrix 0), optional
    int32_t* acc1 = nullptr;   // M x N debug tap (acc of matrix 1), optional
};

// ---- launchers (quant_norm.hip, matmul_skinny.hip, matmul_gemm.hip) ----
hipError_t launch_repack(const uint32_t* words, int rows, int cols, int row_words,
                         Matrix* m, hipStream_t s);
// Microsoft offline U8 layout ((rows/4) x cols bytes) -> loom row-major words
// (rows x ceil(cols/16)).
hipError_t launch_ms_offline_to_words(const uint8_t* packed, int rows, int cols, uint32_t* words,
                                      hipStream_t s);
hipError_t launch_act_quant(const float* x, int ldx, int m, int k, int8_t* xq, int ldq,
                            float* amax, int32_t* xsum, hipStream_t s);
hipError_t launch_act_quant_f64(const double* x, int ldx, int m, int k, int8_t* xq,
                                int ldq, float* amax, int32_t* xsum, hipStream_t s);
// One (NMAT=1) or two (NMAT=2, same shape, EPI_SWIGLU) matrices against the
// same quantized activations.  M is the number of token rows.
hipError_t launch_matmul(const Matrix* w0, const Matrix* w1, const QuantAct& a, int m,
                         const Epilogue& epi, hipStream_t s);
// Same, quantizing fp32 rows x (M x K, row stride K) inside the matmul kernel
// (one launch).  Only for the shapes fused_quant_ok accepts.  xq_tap (M x K)
// and amax_tap (M) optionally receive the quantized rows.
bool fused_quant_ok(int m, int k, const float* x);
hipError_t launch_matmul_fused(const Matrix* w0, const Matrix* w1, const float* x, int m,
                               const Epilogue& epi, int8_t* xq_tap, float* amax_tap,
                               hipStream_t s);
// Row norms a decode matmul can apply to its own input rows before the int8
// quantization (M <= 4 rows), so the norm needs no launch of its own.
enum RowNorm : int {
    NORM_NONE = 0,
    NORM_RMS = 1,        // RMSNormForwardPolymorphic: y = f32((x / rms) * g), fp32 rows
    NORM_INNER_F32 = 2,  // bitNetRMSNormTensorRowWeighted: y = f32(x * scale * w), fp32 rows
    NORM_INNER_F64 = 3,  // bitNetRMSNormFloat64Weighted: y = x * (scale * w), fp64 rows
};
// Whether launch_matmul_norm takes m rows of width k (x16 is the row pointer's
// 16-byte alignment).
bool norm_fused_ok(int m, int k, int strict, bool x16);
// Debug taps of a norm-fused matmul, written by workgroup 0 (all optional):
// the normalized rows (M x K, fp32, or fp64 for NORM_INNER_F64), their int8
// quantization (M x K) and activation absmax (M, floored at 1e-5).
struct NormTaps {
    void* rows = nullptr;
    int8_t* xq = nullptr;
    float* amax = nullptr;
};
// Matmul whose workgroups normalize (mode, strict summation order, gain nw,
// eps) and quantize the rows x (fp32) or x64 (fp64, NORM_INNER_F64)
// themselves.  eps is used as given.  amax_tap (optional, M floats) receives
// the rows' activation absmax.
hipError_t launch_matmul_norm(const Matrix* w0, const Matrix* w1, const float* x, const double* x64,
                              int m, int mode, int strict, const float* nw, double eps,
                              const Epilogue& epi, float* amax_tap, hipStream_t s,
                              const NormTaps* taps = nullptr);

// Inner RMSNorm + requantization of SwiGLU rows (poly/bitnet_cpu.go:893-913 then
// poly/bitnet_cpu.go:97-106).  In place on h (M x n fp32, row stride ldh) unless
// keep_rows is false (then only the int8 rows, amax and sum(xq) are written).
// totals (optional, m doubles of workspace): in strict mode with many rows the
// rows' ordered sums of squares are formed one lane per row first.
hipError_t launch_norm_quant(float* h, int ldh, int m, int n, const float* weight, double eps,
                             int strict, int8_t* hq, int ldq, float* amax, int32_t* xsum,
                             hipStream_t s, bool keep_rows = true, double* totals = nullptr);
// Row norms + requantization of many rows with one wave per row (prefill):
// kRowRms = RMSNorm layer (y = fp32((x / rms) * gain), poly/norm.go:102-138),
// kRowInner = SwiGLU inner norm (x = fp32(x * scale * w), poly/bitnet_cpu.go:893-913),
// kRowInnerF64 = MHA inner norm on fp64 rows (x = x * (scale * w),
// poly/bitnet_cpu.go:868-887), each followed by the int8 quantization of the
// normalized row.  Fast mode sums the squares in the same tree as the
// one-workgroup-per-row kernels (thread t of 256 sums columns t, t + 256, ...;
// then t += t + w for w = 128, 64, ..., 1), so both give the same bits; strict
// mode takes the rows' ordered sums from `totals`.
constexpr int kRowRms = 0, kRowInner = 1, kRowInnerF64 = 2;
struct RowNormArgs {
    const void* x;       // m rows (fp32, fp64 for kRowInnerF64), row stride ldx elements
    long ldx;
    int m, n;
    const float* w;      // gain / weight (n floats) or null (unit weights)
    double eps;
    float* yf;           // kRowRms: y (stride n); kRowInner: x itself (stride ldx); kRowInnerF64: fp32 copy (stride n); or null
    double* keep64;      // kRowInnerF64: x itself (stride ldx), or null
    int8_t* xq;          // quantized rows, stride ldq (zero past n)
    int ldq;
    float* amax;
    int32_t* xsum;
    const double* totals;  // strict: the rows' ordered sums of squares
};
// Launches the one-wave kernel and returns true, or returns false (nothing
// launched) when the rows do not qualify: fewer than 1024 rows, n % 4 != 0,
// rows or outputs not 16-byte aligned, n beyond the kernel's register budget,
// strict without totals, or LOOM_AMD_ROWNORM_WAVE=0.
bool launch_row_norm_wave(int kind, int strict, const RowNormArgs& a, hipStream_t s, hipError_t* e);

// Strict ordered sums of squares of m fp32 rows (one lane per row, in element
// order) into totals when m is large enough and the rows are 16-byte aligned;
// returns false (nothing launched) otherwise.
bool launch_row_sumsq_f32(const float* x, long ldx, int m, int n, double* totals, hipStream_t s,
                          hipError_t* e);

// out[i] = s0 + t[i][0] + t[i][1] + ... + t[i][n-1] in index order (one fp64
// rounding per addition) for m rows of n terms (n <= kMaxStrictNormCols), one
// workgroup of `threads` (64, 256 or 512) per row.
hipError_t launch_ordered_sum_rows(const double* terms, int m, int n, double s0, double* out,
                                   int threads, hipStream_t s);
hipError_t launch_exp_rows(const double* x, long n, double* y, hipStream_t s);

// Per-device scratch arena for the device-resident entry points.
void* scratch(int device, size_t bytes, std::string* err);

const char* kernel_variant(int m);  // name of the matmul path chosen for M rows

// Allocates the GEMM's split-K workspace on a device (once; called when a
// matrix is created there, never by a matmul call).
hipError_t gemm_prepare(int device);

// Tuning overrides (the LOOM_AMD_* variables of the library's tuning table):
// read from the environment once, when the library first needs one, and
// again by loom_amd_reload_tuning(); never per launch (getenv costs host time
// on microsecond launches and is unsafe against setenv on other threads).
// tune_int returns the variable's integer value when it is set and not
// empty, else dflt.
int tune_int(const char* name, int dflt);
void reload_tuning();

}  // namespace lamd
