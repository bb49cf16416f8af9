// matmul_gemm.hip -- ternary x int8 GEMM for many token rows (prefill, M > 64).
//
// Workgroup: 256 threads as 2 (M) x 2 (N) waves; workgroup tile 128 token rows
// x 32*NJ weight rows per matrix; wave tile 64 x 16*NJ (4 x NJ MFMA 16x16x64
// i8 blocks).  Per 256-column K tile:
//   * activations (int8, 128 x 256 B) are staged through LDS, double
//     buffered; rows are padded to 272 B so the 16 lanes that read one MFMA
//     operand column hit 16 different bank groups;
//   * weights go straight from HBM to registers, one 128-bit load per lane per
//     16-row tile (the tile layout), and are unpacked in registers;
//   * the next K tile's loads are issued before the current tile's MFMAs.
// Workgroups are mapped so that each XCD (blockIdx % 8) walks a contiguous run
// of tiles with the weight-row index fastest: consecutive tiles on one XCD share
// the activation tile, which then stays in that XCD's L2.
#include "device_common.hpp"

namespace lamd {

constexpr int kBM = 128;         // token rows per workgroup
constexpr int kLdsRow = 272;     // padded LDS row (bytes) of the activation tile
constexpr int kXcds = 8;

template <int NMAT, int NJ, int PF>
__global__ __launch_bounds__(256, (NJ * NMAT > 4) ? 1 : 2) void gemm_kernel(MatArgs p, int mtiles,
                                                                        int ngroups) {
    static_assert(PF == 1 || PF == 2, "prefetch depth 1 or 2");
    __shared__ __align__(16) int8_t As[2][kBM * kLdsRow];
    constexpr int MI = 4;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wm = wave & 1, wn = wave >> 1;
    const int r = lane & 15, g = lane >> 4;
    const int M = p.e.m;
    const int ktiles = p.ktiles;

    // XCD-aware tile order
    const int total = mtiles * ngroups;
    const int per_xcd = (total + kXcds - 1) / kXcds;
    const int linear = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (linear >= total) return;
    const int mt = linear / ngroups;
    const int ng = linear % ngroups;
    const int m_wg = mt * kBM;
    const int nt0 = (ng * 2 + wn) * NJ;  // wave's first 16-row weight tile

    // ---- weight pointers (tile layout) ----
    const uint4* bptr[NMAT][NJ];
    bool bval[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int nt = nt0 + j;
        bval[j] = nt < p.ntiles;
        const size_t base = (size_t)(bval[j] ? nt : 0) * ktiles * 64 + lane;
        bptr[0][j] = p.w0 + base;
        if (NMAT == 2) bptr[NMAT - 1][j] = p.w1 + base;
    }

    // ---- activation staging: 128 rows x 256 B = 2048 chunks of 16 B, 8 per thread
    auto load_a = [&](int kt, uint4 (&st)[8]) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int lin = c * 256 + tid;
            const int row = lin >> 4;
            const int col = (lin & 15) * 16;
            const int grow = m_wg + row;
            st[c] = grow < M ? *(const uint4*)(p.xq + (size_t)grow * p.ldq + (size_t)kt * kTileCols + col)
                             : uint4{0, 0, 0, 0};
        }
    };
    auto store_a = [&](int buf, const uint4 (&st)[8]) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int lin = c * 256 + tid;
            const int row = lin >> 4;
            const int col = (lin & 15) * 16;
            *(uint4*)(&As[buf][row * kLdsRow + col]) = st[c];
        }
    };
    auto load_b = [&](int kt, uint4 (&b)[NMAT][NJ]) {
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                b[mat][j] = bval[j] ? bptr[mat][j][(size_t)kt * 64] : uint4{0, 0, 0, 0};
    };

    v4i acc[NMAT][MI][NJ];
#pragma unroll
    for (int a = 0; a < NMAT; ++a)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[a][i][j] = v4i{0, 0, 0, 0};

    // Pipeline: LDS holds tile kt; registers hold tile kt+1 ("near") and, with
    // PF == 2, tile kt+2 ("far").
    uint4 st_near[8], st_far[8];
    uint4 b_cur[NMAT][NJ], b_near[NMAT][NJ], b_far[NMAT][NJ];
    load_a(0, st_near);
    load_b(0, b_cur);
    if (ktiles > 1) {
        load_a(1, st_far);
        load_b(1, b_near);
    }
    store_a(0, st_near);
    if (ktiles > 1) {
#pragma unroll
        for (int c = 0; c < 8; ++c) st_near[c] = st_far[c];
    }
    __syncthreads();

    // LDS byte offset of this lane's A operand (M block i, step t): row
    // wm*64 + 16*i + r, column 64*g + 16*t.
    const int a_off = (wm * 64 + r) * kLdsRow + g * 64;

    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        const int kf = kt + PF;  // tile whose loads are issued in this iteration
        if (PF == 2) {
            if (kf < ktiles) {
                load_a(kf, st_far);
                load_b(kf, b_far);
            }
        } else if (kt + 1 < ktiles) {
            load_a(kt + 1, st_near);
            load_b(kt + 1, b_near);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            v4i a[MI];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                a[i] = *(const v4i*)(&As[buf][a_off + i * 16 * kLdsRow + t * 16]);
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const v4i b = unpack_codes(word_of(b_cur[mat][j], t));
#pragma unroll
                    for (int i = 0; i < MI; ++i) acc[mat][i][j] = mfma_i8(a[i], b, acc[mat][i][j]);
                }
        }
        if (kt + 1 < ktiles) {
            store_a(buf ^ 1, st_near);
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int j = 0; j < NJ; ++j) b_cur[mat][j] = b_near[mat][j];
            if (PF == 2) {
#pragma unroll
                for (int c = 0; c < 8; ++c) st_near[c] = st_far[c];
#pragma unroll
                for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) b_near[mat][j] = b_far[mat][j];
            }
        }
        __syncthreads();
    }

    const int m0 = m_wg + wm * 64;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int tok = m0 + 16 * i + 4 * g + v;
            if (tok >= M) continue;
            const RowScale rs = row_scale(p.e, p.e.amax[tok], p.e.xsum[tok]);
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int n = (nt0 + j) * kTileRows + r;
                if (n < p.e.n) epilogue_store(p.e, tok, n, acc[0][i][j][v], acc[NMAT - 1][i][j][v], rs);
            }
        }
}

template <int NMAT, int NJ, int PF>
static hipError_t launch_gemm_t(const MatArgs& p, hipStream_t s) {
    const int mtiles = ceil_div(p.e.m, kBM);
    const int ngroups = ceil_div(p.ntiles, 2 * NJ);
    const int total = mtiles * ngroups;
    const int grid = ceil_div(total, kXcds) * kXcds;
    hipLaunchKernelGGL((gemm_kernel<NMAT, NJ, PF>), dim3(grid), dim3(256), 0, s, p, mtiles, ngroups);
    return hipGetLastError();
}

hipError_t launch_gemm(const MatArgs& p, bool two, hipStream_t s) {
    // Wider weight tiles when there are enough workgroups to fill 256 CUs twice.
    const int mtiles = ceil_div(p.e.m, kBM);
    const bool wide = (size_t)mtiles * ceil_div(p.ntiles, 16) >= 512;
    if (two) return wide ? launch_gemm_t<2, 4, 2>(p, s) : launch_gemm_t<2, 2, 2>(p, s);
    return wide ? launch_gemm_t<1, 8, 2>(p, s) : launch_gemm_t<1, 4, 2>(p, s);
}

}  // namespace lamd
