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
__global__ __launch_bounds__(256, (NJ * NMAT > 4) ? 1 : 2) void gemm128_kernel(MatArgs p, int mtiles,
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
    // wm*64 + 16*i + r, column 64*t + 16*g.
    const int a_off = (wm * 64 + r) * kLdsRow + g * 16;

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
                a[i] = *(const v4i*)(&As[buf][a_off + i * 16 * kLdsRow + t * 64]);
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
static hipError_t launch_gemm128(const MatArgs& p, hipStream_t s) {
    const int mtiles = ceil_div(p.e.m, kBM);
    const int ngroups = ceil_div(p.ntiles, 2 * NJ);
    const int total = mtiles * ngroups;
    const int grid = ceil_div(total, kXcds) * kXcds;
    hipLaunchKernelGGL((gemm128_kernel<NMAT, NJ, PF>), dim3(grid), dim3(256), 0, s, p, mtiles, ngroups);
    return hipGetLastError();
}

constexpr int kBM3 = 256;
constexpr int kRow3 = 144;
// dword 3 of a raw (untyped, unswizzled) gfx9 buffer resource
constexpr int kBufferWord3 = 0x00020000;

// ------------------------------------------------------------------------
// gemm512: 512-thread workgroups (2 x 4 waves), workgroup tile 256 token rows
// x 256/NMAT weight rows per matrix, wave tile 128 x 64/NMAT.  The activation
// stage (256 x 128 B) is shared by four N waves; each thread stages only 64 B
// of it, which leaves registers for loads issued two stages ahead (register
// double buffer) while LDS stays double buffered.
// ------------------------------------------------------------------------

template <int NMAT, int EPI>
__global__ __launch_bounds__(512, 1) void gemm512_kernel(MatArgs p, int mtiles, int ngroups) {
    constexpr int MI = 8;
    constexpr int NJ = 4 / NMAT;
    __shared__ __align__(16) int8_t As[2][kBM3 * kRow3];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wm = wave & 1, wn = wave >> 1;
    const int r = lane & 15, g = lane >> 4;
    const int M = p.e.m;
    const int ktiles = p.ktiles;
    const int nstages = 2 * ktiles;

    const int total = mtiles * ngroups;
    const int per_xcd = (total + kXcds - 1) / kXcds;
    const int linear = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (linear >= total) return;
    const int mt = linear / ngroups;
    const int ng = linear % ngroups;
    const int m_wg = mt * kBM3;
    const int nt0 = (ng * 4 + wn) * NJ;

    const __amdgpu_buffer_rsrc_t wres0 =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.w0, 0, 0x7fffffff, kBufferWord3);
    const __amdgpu_buffer_rsrc_t wres1 =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.w1, 0, 0x7fffffff, kBufferWord3);
    const __amdgpu_buffer_rsrc_t ares =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.xq, 0, 0x7fffffff, kBufferWord3);
    int woff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int nt = min(nt0 + j, p.ntiles - 1);
        woff[j] = (nt * ktiles * 64 + lane) * 16;
    }
    // chunk c (0..3) of thread tid -> row 64*c + (tid>>3), 16-byte column tid&7
    int aoff_g[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int row = min(m_wg + 64 * c + (tid >> 3), M - 1);
        aoff_g[c] = row * p.ldq + (tid & 7) * 16;
    }
    const int aoff0 = (tid >> 3) * kRow3 + (tid & 7) * 16;
    // Every stage loads, unconditionally, its activation chunk (4 x 16 B per
    // thread) and the 8-byte weight half it needs, two stages ahead of use
    // (indices clamped at the end: the extra loads are never consumed).  The
    // loop body has no branches, so the wait counters see a fixed pattern:
    // data issued two stages earlier is complete without draining new loads.
    uint4 st_near[4], st_far[4];
    uint2 b_cur[NMAT][NJ], b_near[NMAT][NJ], b_far[NMAT][NJ];
    auto load_a = [&](int stage, uint4 (&st)[4]) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            st[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ares, aoff_g[c], stage * 128, 0));
    };
    auto store_a = [&](int buf, const uint4 (&st)[4]) {
#pragma unroll
        for (int c = 0; c < 4; ++c) *(uint4*)(&As[buf][aoff0 + c * 64 * kRow3]) = st[c];
    };
    // weights of stage s: words 2*(s&1), 2*(s&1)+1 of K tile s>>1
    auto load_b = [&](int stage, uint2 (&b)[NMAT][NJ]) {
        const int soff = (stage >> 1) * 1024 + (stage & 1) * 8;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            b[0][j] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wres0, woff[j], soff, 0));
            if (NMAT == 2)
                b[NMAT - 1][j] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wres1, woff[j], soff, 0));
        }
    };

    v4i acc[NMAT][MI][NJ];
#pragma unroll
    for (int a = 0; a < NMAT; ++a)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[a][i][j] = v4i{0, 0, 0, 0};

    const int last = nstages - 1;
    load_a(0, st_far);
    load_b(0, b_cur);
    load_a(min(1, last), st_near);
    load_b(min(1, last), b_near);
    store_a(0, st_far);
    __syncthreads();

    const int a_off = (wm * 128 + r) * kRow3 + g * 16;
    for (int s = 0; s < nstages; ++s) {
        const int buf = s & 1;
        load_a(min(s + 2, last), st_far);
        load_b(min(s + 2, last), b_far);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            v4i b[NMAT][NJ];
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int j = 0; j < NJ; ++j) b[mat][j] = unpack_codes(t == 0 ? b_cur[mat][j].x : b_cur[mat][j].y);
            v4i a[MI];
#pragma unroll
            for (int i = 0; i < MI; ++i) a[i] = *(const v4i*)(&As[buf][a_off + i * 16 * kRow3 + t * 64]);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) acc[mat][i][j] = mfma_i8(a[i], b[mat][j], acc[mat][i][j]);
        }
        store_a(buf ^ 1, st_near);  // stage s+1 (a clamped copy after the last stage: unused)
#pragma unroll
        for (int c = 0; c < 4; ++c) st_near[c] = st_far[c];
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                b_cur[mat][j] = b_near[mat][j];
                b_near[mat][j] = b_far[mat][j];
            }
        __syncthreads();
    }

    const int m0 = m_wg + wm * 128;
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
                if (n >= p.e.n) continue;
                if (EPI == 0) {
                    p.e.out[(size_t)tok * p.e.ldo + n] = (float)((double)(acc[0][i][j][v] - rs.xs) * rs.os0);
                } else {
                    epilogue_store(p.e, tok, n, acc[0][i][j][v], acc[NMAT - 1][i][j][v], rs);
                }
            }
        }
}

template <int NMAT, int EPI>
static hipError_t launch_gemm512(const MatArgs& p, hipStream_t s) {
    const int mtiles = ceil_div(p.e.m, kBM3);
    const int ngroups = ceil_div(p.ntiles, 4 * (4 / NMAT));
    const int total = mtiles * ngroups;
    const int grid = ceil_div(total, kXcds) * kXcds;
    hipLaunchKernelGGL((gemm512_kernel<NMAT, EPI>), dim3(grid), dim3(512), 0, s, p, mtiles, ngroups);
    return hipGetLastError();
}

static bool plain_dense(const EpiDev& e) {
    return e.kind == EPI_DENSE && !e.bias0 && !e.residual && !e.post && !e.acc0;
}

hipError_t launch_gemm(const MatArgs& p, bool two, hipStream_t s) {
    // 256 x 256 workgroup tiles from 128 of them up (one per CU, eight waves
    // each); 128-row tiles below, where more workgroups are needed.
    const size_t big = (size_t)ceil_div(p.e.m, kBM3) * ceil_div(p.ntiles, 16);
    if (big >= 128) {
        if (two) return launch_gemm512<2, 1>(p, s);
        return plain_dense(p.e) ? launch_gemm512<1, 0>(p, s) : launch_gemm512<1, 1>(p, s);
    }
    return two ? launch_gemm128<2, 2, 2>(p, s) : launch_gemm128<1, 4, 2>(p, s);
}

}  // namespace lamd
