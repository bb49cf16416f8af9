// matmul_gemm.hip -- ternary x int8 GEMM for many token rows (prefill, M > 64).
#include <mutex>
#include <vector>

#include "device_common.hpp"

namespace lamd {

constexpr int kXcds = 8;

// Split-K workspace of one device: int32 partial accumulators of up to
// kSplitSlots workgroups (kSplitSlotInts each) and one arrival counter per
// output tile.  The counters start at zero and the last workgroup of a tile
// sets its counter back to zero, so no launch clears them.  Allocated when a
// matrix is created on the device, never inside a matmul call (which may be
// under stream capture); without it the GEMM does not split.  Split launches
// that overlap on one device would share it: they are issued on one stream.
constexpr int kSplitSlotInts = 64 * 256;  // 64-token tiles: 64 accumulators x 256 threads
constexpr int kSplitSlots = 768;
constexpr int kSplitTiles = 1024;
struct SplitWs {
    int32_t* part = nullptr;
    unsigned* ctr = nullptr;
    int32_t* sacc = nullptr;  // small-M split: accumulators, zero between launches
    unsigned* sctr = nullptr;  // small-M split: arrival counters, zero between launches
};
static std::mutex g_split_mu;
static std::vector<SplitWs> g_split;

hipError_t gemm_prepare(int device) {
    std::lock_guard<std::mutex> lock(g_split_mu);
    if ((int)g_split.size() <= device) g_split.resize(device + 1);
    SplitWs& w = g_split[device];
    if (w.part) return hipSuccess;
    int32_t* part = nullptr;
    unsigned* ctr = nullptr;
    int32_t* sacc = nullptr;
    unsigned* sctr = nullptr;
    hipError_t e = hipMalloc(&part, (size_t)kSplitSlots * kSplitSlotInts * 4);
    if (e == hipSuccess) e = hipMalloc(&ctr, (size_t)kSplitTiles * 4);
    if (e == hipSuccess) e = hipMemset(ctr, 0, (size_t)kSplitTiles * 4);
    if (e == hipSuccess) e = hipMalloc(&sacc, (size_t)kSmallSplitInts * 4);
    if (e == hipSuccess) e = hipMemset(sacc, 0, (size_t)kSmallSplitInts * 4);
    if (e == hipSuccess) e = hipMalloc(&sctr, (size_t)kSmallSplitGroups * 4);
    if (e == hipSuccess) e = hipMemset(sctr, 0, (size_t)kSmallSplitGroups * 4);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        if (part) (void)hipFree(part);
        if (ctr) (void)hipFree(ctr);
        if (sacc) (void)hipFree(sacc);
        if (sctr) (void)hipFree(sctr);
        return e;
    }
    w.part = part;
    w.ctr = ctr;
    w.sacc = sacc;
    w.sctr = sctr;
    return hipSuccess;
}

SmallSplitWs small_split_ws(int device) {
    std::lock_guard<std::mutex> lock(g_split_mu);
    if (device >= (int)g_split.size()) return SmallSplitWs{};
    return SmallSplitWs{g_split[device].sacc, g_split[device].sctr};
}

static SplitWs split_ws(int device) {
    std::lock_guard<std::mutex> lock(g_split_mu);
    return device < (int)g_split.size() ? g_split[device] : SplitWs{};
}

// Grid of one GEMM launch: mtiles x ngroups output tiles, each split into
// ksplit ranges of `sps` K stages (the last range may be shorter).
struct GemmGrid {
    int mtiles, ngroups, ksplit, sps;
    int group;  // token tiles per group of the tile order (0: weight-row group fastest)
    int32_t* part;
    unsigned* ctr;
};

// ------------------------------------------------------------------------
// gemm_lds_kernel: v_mfma_i32_32x32x32_i8, which issues int8 at twice the
// rate of the 16x16x64 form on gfx950 (measured: 4.5 vs 2.5 POPS sustained).
// 256 threads as 4 waves along N; workgroup tile 32*MI tokens x 256/NMAT
// weight rows per matrix, wave tile 32*MI tokens x 64/NMAT weight rows (MI x
// NJ blocks of 32 x 32); K stages of 256 columns (one K tile).  MI = 2
// (64-token tiles, three workgroups per CU) serves mid-size M and split K;
// MI = 4 (128-token tiles, two per CU) feeds each unpacked weight word to
// four MFMAs instead of two, which pays once the grid is large.
// Tile order: workgroups are mapped so that each XCD (blockIdx % 8) walks a
// contiguous run of tiles, in groups of `group` token tiles with the
// weight-row group fastest inside a group: consecutive tiles on one XCD share
// activation and weight tiles, which then stay in that XCD's L2.
// Weights come straight from the 16-row tile layout: lane l takes weight row
// l&31 of its 32-row block (tile (l>>4)&1, row l&15) and loads the words of
// tile lanes (l&15) + 16h and (l&15) + 16h + 32 (h = l>>5), which hold the K
// chunks 4t + h and 4t + 2 + h of every 256-column tile.  MFMA step q of a
// stage pairs chunk c and c + 1 (c = 0, 4, 2, 6 within the stage) across the
// two K halves, so the eight words a lane holds per tile are exactly its
// eight K steps.
// Activations: the stages are copied global -> LDS by the memory units
// (buffer_load ... lds, 16 bytes a lane), so no VGPRs stage them and the
// A-operand reads run ahead of the MFMAs.  MI = 2 keeps three stage buffers
// (stage s + 2 copied, with its weight words loaded into the third register
// set, while stage s is computed); MI = 4 keeps two (stage s + 1).  One
// barrier per stage both publishes the next stage and frees the buffer just
// read.  Each wave waits for its own copies (vmcnt) before that barrier; a
// bare s_barrier is used because __syncthreads' release fence would wait for
// every outstanding copy.
// Stage buffer layout: 32*MI rows x 16 chunks of 16 bytes, row R at R*256,
// its logical chunk ch at physical chunk ch ^ (R & 15), so the 8 (or 16) rows
// a group of lanes reads in one MFMA step fall in distinct banks; the copies
// gather each row's chunks in that order (each copy instruction still reads
// whole 256-byte row segments).
// Split K (ksplit > 1, MI = 2 only): workgroup (tile, r) sums K stages
// [r*sps, (r+1)*sps), stores its int32 accumulators to its workspace slot,
// and the last of the tile's workgroups to arrive (a device-scope counter)
// adds the other slots to its own -- integer adds, so the result is the same
// in any order -- and runs the epilogue.
// The epilogue stores straight from the accumulators: per instruction the
// two half-waves write 128 contiguous bytes of two rows.
// EPI: 0 = plain dense (fp32 out only), 1 + EPI_DENSE / EPI_SWIGLU / EPI_ACC =
// that epilogue kind with its optional bias, residual, activation and taps.
// ------------------------------------------------------------------------

#ifndef LAMD_G64_AHEAD
#define LAMD_G64_AHEAD 2
#endif

// The stage buffers are distinct arrays and these helpers take
// restrict pointers, so the compiler's wait before an LDS read covers only
// the copies into the buffer being read.
__device__ __forceinline__ void g64_copy(__amdgpu_buffer_rsrc_t r, int8_t* __restrict__ dst, int voff,
                                         int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff,
                                             soff, 0, 0);
}
__device__ __forceinline__ v4i g64_read(const int8_t* __restrict__ src, int off) {
    return *(const v4i*)(src + off);
}
// s_waitcnt vmcnt(N) lgkmcnt(0): at most N vector-memory operations of this
// wave outstanding (its older stage copies have landed in LDS) and none of
// its LDS operations (its reads of the buffer that the barrier after this
// wait hands to the next copy have returned).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}
// s_waitcnt lgkmcnt(0) only (vmcnt and expcnt at their maxima)
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

template <int NMAT, int EPI, int MI, int NJ>
__global__ __launch_bounds__(256, 2) void gemm_lds_kernel(MatArgs p, GemmGrid gg) {
    static_assert(NJ >= 1 && NJ * NMAT <= 2, "32-row weight blocks per wave and matrix");
    constexpr int BM = 32 * MI;
    constexpr int NA = BM / 16;  // copies per thread per stage
    constexpr int NSTEP = 8;     // MFMA K steps per 256-column stage
    constexpr int NB = NMAT * NJ * 2;  // weight loads per thread per stage
    static_assert(MI == 2 || MI == 4, "64- or 128-token tiles");
    __shared__ __align__(16) int8_t As0[BM * 256];
    __shared__ __align__(16) int8_t As1[BM * 256];
    __shared__ __align__(16) int8_t As2[MI == 2 ? BM * 256 : 16];  // (128-token tiles: two buffers)
    __shared__ int s_last;
    __shared__ double s_os0[BM], s_os1[NMAT == 2 ? BM : 1];
    __shared__ int s_xs[BM];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int wn = wave;
    const int l32 = lane & 31, h = lane >> 5;
    const int M = p.e.m;
    const int ktiles = p.ktiles;
    const int S = gg.ksplit;

    const int total = gg.mtiles * gg.ngroups * S;
    const int per_xcd = (total + kXcds - 1) / kXcds;
    const int linear = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (linear >= total) return;
    const int tile = linear / S;
    const int split = linear - tile * S;
    int mt, ng;
    if (gg.group > 0) {
        const int per_group = gg.group * gg.ngroups;
        const int g0 = tile / per_group;
        const int first = g0 * gg.group;
        const int gsz = min(gg.mtiles - first, gg.group);
        const int in = tile - g0 * per_group;
        mt = first + in % gsz;
        ng = in / gsz;
    } else {
        mt = tile / gg.ngroups;
        ng = tile % gg.ngroups;
    }
    const int st0 = split * gg.sps;
    const int st1 = min(st0 + gg.sps, ktiles);
    const int last = st1 - 1;
    const int m_wg = mt * BM;
    const int nb0 = (ng * 4 + wn) * NJ;  // wave's first 32-row weight block
    for (int t = tid; t < BM; t += 256) {
        const int tok = min(m_wg + t, M - 1);
        const RowScale rs = row_scale(p.e, p.e.amax[tok], p.e.xsum[tok]);
        s_os0[t] = rs.os0;
        if (NMAT == 2) s_os1[t] = rs.os1;
        s_xs[t] = rs.xs;
    }

    const __amdgpu_buffer_rsrc_t wres0 =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.w0, 0, 0x7fffffff, kBufferWord3);
    const __amdgpu_buffer_rsrc_t wres1 =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.w1, 0, 0x7fffffff, kBufferWord3);
    const __amdgpu_buffer_rsrc_t ares =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.xq, 0, 0x7fffffff, kBufferWord3);
    int woff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int nt = min(2 * (nb0 + j) + ((lane >> 4) & 1), p.ntiles - 1);
        woff[j] = (nt * ktiles * 64 + (lane & 15) + 16 * h) * 16;
    }
    // copy c of this lane fills physical chunk P = 256c + 64*wave + lane of a
    // stage buffer: row P/16, physical chunk P%16 = logical chunk
    // (P%16) ^ (row%16) of that token row
    int aoff_g[NA];
#pragma unroll
    for (int c = 0; c < NA; ++c) {
        const int P = 256 * c + 64 * wave + lane;
        const int r = P >> 4;
        const int lc = (P & 15) ^ (r & 15);
        aoff_g[c] = min(m_wg + r, M - 1) * p.ldq + lc * 16;
    }
    auto issue = [&](int8_t* buf, int stage, uint32_t (&b)[NMAT][NJ][2][4]) {
#pragma unroll
        for (int c = 0; c < NA; ++c) g64_copy(ares, buf + c * 4096 + wave * 1024, aoff_g[c], stage * 256);
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const __amdgpu_buffer_rsrc_t r = mat == 0 ? wres0 : wres1;
                    const uint4 w = __builtin_bit_cast(
                        uint4, __builtin_amdgcn_raw_buffer_load_b128(r, woff[j] + 512 * u, stage * 1024, 0));
                    b[mat][j][u][0] = w.x;
                    b[mat][j][u][1] = w.y;
                    b[mat][j][u][2] = w.z;
                    b[mat][j][u][3] = w.w;
                }
    };

    v16i acc[NMAT][MI][NJ];
#pragma unroll
    for (int a = 0; a < NMAT; ++a)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[a][i][j] = v16i{};

    // lane's A rows l32 and 32 + l32 (immediate +8192); step with chunk pair
    // (c0, c0 + 1) reads logical chunk c0 + h = c0 ^ h at physical chunk
    // c0 ^ h ^ (l32 & 15)
    const int abase = l32 * 256 + ((h ^ (l32 & 15)) << 4);
    auto compute = [&](const int8_t* buf, const uint32_t (&bw)[NMAT][NJ][2][4]) {
#pragma unroll
        for (int idx = 0; idx < NSTEP; ++idx) {
            const int hh = idx >> 2, q = idx & 3;
            const int c0 = hh * 8 + (q & 1) * 4 + (q >> 1) * 2;
            const int off = abase ^ (c0 << 4);
            v4i a[MI];
#pragma unroll
            for (int i = 0; i < MI; ++i) a[i] = g64_read(buf, off + i * 8192);
            v4i b[NMAT][NJ];
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int j = 0; j < NJ; ++j) b[mat][j] = unpack_codes(bw[mat][j][q >> 1][2 * hh + (q & 1)]);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) acc[mat][i][j] = mfma32_i8(a[i], b[mat][j], acc[mat][i][j]);
        }
    };

    // Instruction order of one region between barriers: stage s+2's copies
    // and weight loads first, the A reads of a step LAMD_G64_AHEAD steps
    // before its MFMAs, each MFMA followed by a share of the next step's
    // unpack.
    constexpr int NMF = MI * NJ * NMAT;         // MFMAs per step
    constexpr int NUP = NMAT * NJ * 7;          // unpack VALU per step
    constexpr int VPM = (NUP + NMF - 1) / NMF;  // VALU per MFMA slot
    auto region_order = [&]() {
        __builtin_amdgcn_sched_group_barrier(0x020, NA + NB, 0);
#pragma unroll
        for (int k = 0; k < LAMD_G64_AHEAD; ++k) __builtin_amdgcn_sched_group_barrier(0x100, MI, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, NUP, 0);
#pragma unroll
        for (int idx = 0; idx < NSTEP; ++idx) {
#pragma unroll
            for (int m = 0; m < NMF; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
            }
            if (idx + LAMD_G64_AHEAD < NSTEP) __builtin_amdgcn_sched_group_barrier(0x100, MI, 0);
        }
    };
    // Vector-memory operations that may still be outstanding when a stage's
    // copies must have landed: the whole issue of the stage after it.  (The
    // scheduler may place an issue's weight loads before or after its
    // copies, so a count that relied on the order inside one issue could let
    // copies of the stage about to be read through.)
    constexpr int kAfter = NA + NB;
    uint32_t bw0[NMAT][NJ][2][4], bw1[NMAT][NJ][2][4], bw2[NMAT][NJ][2][4];
    if constexpr (MI == 4) {
        // 128-token tiles: two 32 KB stage buffers (two workgroups per CU),
        // stage s+1 copied while stage s is computed
        // (every wait counts all of the next stage's loads: the scheduler may
        // place its weight loads before or after its copies)
        issue(As0, st0, bw0);
        wait_vm_lgkm0<0>();  // (lgkmcnt also covers the per-token constants)
        __builtin_amdgcn_s_barrier();
        int s = st0;
        for (; s + 1 < st1; s += 2) {
            issue(As1, s + 1, bw1);
            compute(As0, bw0);
            region_order();
            wait_vm_lgkm0<0>();  // stage s+1's copies have landed; As0's reads returned
            __builtin_amdgcn_s_barrier();
            issue(As0, min(s + 2, last), bw0);
            compute(As1, bw1);
            region_order();
            wait_vm_lgkm0<0>();
            __builtin_amdgcn_s_barrier();
        }
        if (s < st1) compute(As0, bw0);
    } else {
    issue(As0, st0, bw0);
    issue(As1, min(st0 + 1, last), bw1);
    wait_vm_lgkm0<kAfter>();  // (lgkmcnt also covers the per-token constants)
    __builtin_amdgcn_s_barrier();
    int s = st0;
    for (; s + 2 < st1; s += 3) {
        issue(As2, min(s + 2, last), bw2);
        compute(As0, bw0);
        region_order();
        wait_vm_lgkm0<kAfter>();
        __builtin_amdgcn_s_barrier();
        issue(As0, min(s + 3, last), bw0);
        compute(As1, bw1);
        region_order();
        wait_vm_lgkm0<kAfter>();
        __builtin_amdgcn_s_barrier();
        issue(As1, min(s + 4, last), bw1);
        compute(As2, bw2);
        region_order();
        wait_vm_lgkm0<kAfter>();
        __builtin_amdgcn_s_barrier();
    }
    if (s < st1) {
        compute(As0, bw0);
        if (s + 1 < st1) {
            wait_vm_lgkm0<0>();  // stage s+1's copies and weights (the last issued)
            __builtin_amdgcn_s_barrier();
            compute(As1, bw1);
        }
    }
    }
    wait_vm_lgkm0<0>();  // no copy may still be writing LDS when the workgroup ends

    if (MI == 2 && S > 1) {
        // Slot layout: 16-byte group q (values 4q .. 4q+3) of accumulator
        // block b of thread t at int offset ((b*4 + q)*256 + t)*4, so each
        // store or load instruction of the workgroup covers 4 KB in one run.
        const __amdgpu_buffer_rsrc_t mine =
            buffer_rsrc(gg.part + (size_t)linear * kSplitSlotInts, kSplitSlotInts * 4);
#pragma unroll
        for (int a = 0; a < NMAT; ++a)
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const v16i& c = acc[a][i][j];
                        const u32x4 w = {(unsigned)c[4 * q], (unsigned)c[4 * q + 1], (unsigned)c[4 * q + 2],
                                         (unsigned)c[4 * q + 3]};
                        buffer_store16_sc1(w, mine, (uint32_t)(((((a * MI + i) * NJ + j) * 4 + q) * 256 + tid) * 16));
                    }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            s_last = __hip_atomic_fetch_add(&gg.ctr[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (unsigned)(S - 1);
        }
        __syncthreads();
        if (!s_last) return;
        // one slot at a time, its 16 loads issued before any add
        for (int o = 0; o < S; ++o) {
            if (o == split) continue;
            const __amdgpu_buffer_rsrc_t src =
                buffer_rsrc(gg.part + (size_t)(tile * S + o) * kSplitSlotInts, kSplitSlotInts * 4);
            u32x4 t[NMAT][MI][NJ][4];
#pragma unroll
            for (int a = 0; a < NMAT; ++a)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            t[a][i][j][q] =
                                buffer_load16_sc1(src, (uint32_t)(((((a * MI + i) * NJ + j) * 4 + q) * 256 + tid) * 16));
#pragma unroll
            for (int a = 0; a < NMAT; ++a)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
#pragma unroll
                            for (int r = 0; r < 4; ++r) acc[a][i][j][4 * q + r] += (int)t[a][i][j][q][r];
        }
        if (tid == 0) __hip_atomic_store(&gg.ctr[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    static_assert(MI != 2 || NMAT * MI * NJ * 16 * 256 <= kSplitSlotInts, "a split slot holds one 64-token tile");

    // Epilogue from the accumulators: value v of block (i, j) is token row
    // 32i + 8(v/4) + 4h + v%4, output column (nb0 + j)*32 + l32.
    // (the test covers the workgroup's whole tile, not this wave's columns:
    // every wave of the workgroup takes this path and meets its barrier.
    // 128-token tiles only: on the 64-token tiles of mid-size M it measured
    // slower than storing from the accumulators.)
    if (EPI == 0 && MI == 4 && m_wg + BM <= M && (ng * 4 + 4) * NJ * 32 <= p.e.n && p.e.ldo % 4 == 0 &&
        ((uintptr_t)p.e.out & 15) == 0) {
        // plain Dense on a full tile with 16-byte aligned rows: each 32 x 32
        // block of a wave is written to a wave-private LDS tile in the
        // accumulator layout and read back as four adjacent columns per lane,
        // so one store instruction writes 8 whole 128-byte row segments with
        // 16 bytes a lane (a quarter of the store instructions of storing
        // from the accumulators).  The stage buffers hold the tiles: every
        // wave has finished its MFMA operand reads at the barrier.
        constexpr int TP = 40;  // tile pitch (floats): 16-byte rows; the two half-waves' rows in disjoint banks
        static_assert(MI != 4 || 4 * 32 * TP * 4 <= BM * 256, "epilogue tiles");
        __builtin_amdgcn_s_barrier();
        float* tl = (float*)As0 + wave * 32 * TP;
        const int ldo = p.e.ldo;
        const double* os_l = s_os0 + 4 * h;
        const int* xs_l = s_xs + 4 * h;
        // read-back: row rr + 8k, columns cc .. cc + 3; each 16-lane group reads
        // rows r and r + 4, whose segments lie 32 banks apart at pitch 40
        const int rr = (lane >> 4) + 4 * ((lane >> 3) & 1), cc = (lane & 7) * 4;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int t = 32 * i + 8 * g + u;  // this lane's row: t + 4h
                        tl[(8 * g + 4 * h + u) * TP + l32] =
                            (float)((double)(acc[0][i][j][4 * g + u] - xs_l[t]) * os_l[t]);
                    }
                wait_lgkm0();  // the wave's tile writes have landed
                float* orow = p.e.out + (size_t)(m_wg + 32 * i + rr) * ldo + (nb0 + j) * 32 + cc;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 v = *(const float4*)&tl[(rr + 8 * k) * TP + cc];
                    store16_nt(orow + (size_t)(8 * k) * ldo, v.x, v.y, v.z, v.w);
                }
                wait_lgkm0();  // read back before the next block's writes
            }
        return;
    }
    if (EPI == 0 && m_wg + BM <= M && (nb0 + NJ) * 32 <= p.e.n) {
        // plain Dense on a full tile: no row or column tests; each store
        // takes a wave-uniform row pointer plus this lane's 32-bit offset,
        // and the per-token constants come from LDS at immediate offsets
        const int ldo = p.e.ldo;
        const int loff = 4 * h * ldo + nb0 * 32 + l32;
        const double* os_l = s_os0 + 4 * h;
        const int* xs_l = s_xs + 4 * h;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int t = 32 * i + 8 * g + u;  // this lane's row: t + 4h
                    float* rowp = p.e.out + (size_t)(m_wg + t) * ldo;
                    const double os0 = os_l[t];
                    const int xs = xs_l[t];
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        __builtin_nontemporal_store((float)((double)(acc[0][i][j][4 * g + u] - xs) * os0),
                                                    &rowp[loff + 32 * j]);
                }
        return;
    }
    if (EPI != 0 && MI == 4 && m_wg + BM <= M && (ng * 4 + 4) * NJ * 32 <= p.e.n &&
        (EPI == 1 + EPI_ACC ? p.e.n % 4 == 0 && ((uintptr_t)p.e.acc0 & 15) == 0
                            : !p.e.acc0 && !p.e.acc1 && !p.e.post && p.e.ldo % 4 == 0 &&
                                  ((uintptr_t)p.e.out & 15) == 0 &&
                                  (!p.e.residual || ((uintptr_t)p.e.residual & 15) == 0))) {
        // the other epilogues on a full 128-token tile, through the same
        // wave-private LDS tiles as the plain Dense one (workgroup-uniform
        // test, one barrier): in the accumulator layout each value is
        // rescaled (+ bias) to its fp32 pre-residual value (SwiGLU: the gate
        // product; EPI_ACC: the int32 accumulator's bits); read back as four
        // adjacent columns of a row, the residual (one 16-byte load) and the
        // stores follow in the reference's order.  (With an activation copy
        // or accumulator taps the accumulators would stay live across their
        // code and spill: those take the path below.)
        constexpr int TP = 40;
        static_assert(MI != 4 || 4 * 32 * TP * 4 <= BM * 256, "epilogue tiles");
        __builtin_amdgcn_s_barrier();
        float* tl = (float*)As0 + wave * 32 * TP;
        const int ldo = p.e.ldo, ldn = p.e.n;
        const double* os0_l = s_os0 + 4 * h;
        const double* os1_l = NMAT == 2 ? s_os1 + 4 * h : s_os0;
        const int* xs_l = s_xs + 4 * h;
        const bool has_res = EPI == 1 + EPI_DENSE && p.e.residual;
        const int rr = (lane >> 4) + 4 * ((lane >> 3) & 1), cc = (lane & 7) * 4;
        static_for<NJ>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const int col = (nb0 + j) * 32 + l32;
            const float bias0 = EPI != 1 + EPI_ACC && p.e.bias0 ? p.e.bias0[col] : 0.0f;
            const float bias1 = NMAT == 2 && p.e.bias1 ? p.e.bias1[col] : 0.0f;
            static_for<MI>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int t = 32 * i + 8 * g + u;  // this lane's row: t + 4h
                        const int xs = xs_l[t];
                        const int a0 = acc[0][i][j][4 * g + u] - xs;
                        float v;
                        if (EPI == 1 + EPI_ACC) {
                            v = __int_as_float(a0);
                        } else if (EPI == 1 + EPI_SWIGLU) {
                            const int a1 = acc[NMAT - 1][i][j][4 * g + u] - xs;
                            const double gg0 = (double)a0 * os0_l[t] + (p.e.bias0 ? (double)bias0 : 0.0);
                            const double uu = (double)a1 * os1_l[t] + (p.e.bias1 ? (double)bias1 : 0.0);
                            v = (float)gate_product(gg0, uu, p.e.activation);
                        } else {
                            double d = (double)a0 * os0_l[t];
                            if (p.e.bias0) d = d + (double)bias0;
                            v = (float)d;
                        }
                        tl[(8 * g + 4 * h + u) * TP + l32] = v;
                    }
                wait_lgkm0();  // the wave's tile writes have landed
                const size_t row0 = (size_t)(m_wg + 32 * i + rr);
                const int c0 = (nb0 + j) * 32 + cc;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 v = *(const float4*)&tl[(rr + 8 * k) * TP + cc];
                    const size_t row = row0 + 8 * k;
                    if (EPI == 1 + EPI_ACC) {
                        *(int4*)(p.e.acc0 + row * ldn + c0) =
                            make_int4(__float_as_int(v.x), __float_as_int(v.y), __float_as_int(v.z), __float_as_int(v.w));
                    } else if (EPI == 1 + EPI_SWIGLU) {
                        *(float4*)(p.e.out + row * ldo + c0) = v;
                    } else {
                        float4 o = v;
                        if (has_res) {
                            const float4 r4 = *(const float4*)(p.e.residual + row * ldo + c0);
                            o = make_float4(o.x + r4.x, o.y + r4.y, o.z + r4.z, o.w + r4.w);
                        }
                        *(float4*)(p.e.out + row * ldo + c0) = o;
                    }
                }
                wait_lgkm0();  // read back before the next block's writes
            });
        });
        return;
    }
    if (EPI != 0 && m_wg + BM <= M && (nb0 + NJ) * 32 <= p.e.n) {
        // every other epilogue on a full tile: the same branch-free row walk
        // (wave-uniform row offsets, this lane's column), residual loads of a
        // row group issued before its stores
        const int ldo = p.e.ldo, ldn = p.e.n;
        const int col = nb0 * 32 + l32;
        float bias0[NJ], bias1[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            bias0[j] = p.e.bias0 ? p.e.bias0[col + 32 * j] : 0.0f;
            bias1[j] = NMAT == 2 && p.e.bias1 ? p.e.bias1[col + 32 * j] : 0.0f;
        }
        const bool has_res = EPI == 1 + EPI_DENSE && p.e.residual;
        const double* os0_l = s_os0 + 4 * h;
        const double* os1_l = NMAT == 2 ? s_os1 + 4 * h : s_os0;
        const int* xs_l = s_xs + 4 * h;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float res[4][NJ];
                if (has_res) {
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const float* rrow = p.e.residual + (size_t)(m_wg + 32 * i + 8 * g + u) * ldo;
#pragma unroll
                        for (int j = 0; j < NJ; ++j) res[u][j] = rrow[4 * h * ldo + col + 32 * j];
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int t = 32 * i + 8 * g + u;  // this lane's row: t + 4h
                    const size_t row = (size_t)(m_wg + t);
                    const double os0 = os0_l[t];
                    const double os1 = NMAT == 2 ? os1_l[t] : 0.0;
                    const int xs = xs_l[t];
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const int raw0 = acc[0][i][j][4 * g + u];
                        const int raw1 = NMAT == 2 ? acc[NMAT - 1][i][j][4 * g + u] : raw0;
                        const int a0 = raw0 - xs;
                        const int c = 4 * h * ldn + col + 32 * j;  // (acc taps: row pitch N)
                        const int co = 4 * h * ldo + col + 32 * j;
                        if (p.e.acc0) p.e.acc0[row * ldn + c] = a0;
                        if (EPI == 1 + EPI_ACC) continue;
                        if (EPI == 1 + EPI_SWIGLU) {
                            const int a1 = raw1 - xs;
                            if (p.e.acc1) p.e.acc1[row * ldn + c] = a1;
                            const double gg0 = (double)a0 * os0 + (p.e.bias0 ? (double)bias0[j] : 0.0);
                            const double uu = (double)a1 * os1 + (p.e.bias1 ? (double)bias1[j] : 0.0);
                            p.e.out[row * ldo + co] = (float)gate_product(gg0, uu, p.e.activation);
                        } else {
                            double d = (double)a0 * os0;
                            if (p.e.bias0) d = d + (double)bias0[j];
                            float v = (float)d;
                            if (has_res) v = v + res[u][j];
                            p.e.out[row * ldo + co] = v;
                            if (p.e.post) p.e.post[row * ldo + co] = activate_f32(v, p.e.activation);
                        }
                    }
                }
            }
        return;
    }
    // (general case) Residual loads of four rows are issued before their stores.
    float bias0[NJ], bias1 = 0.0f;
    bool ncol[NJ];
    int ncl[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int n = (nb0 + j) * 32 + l32;
        ncol[j] = n < p.e.n;
        ncl[j] = min(n, p.e.n - 1);
        bias0[j] = EPI && p.e.bias0 ? p.e.bias0[ncl[j]] : 0.0f;
    }
    if (EPI && NMAT == 2 && p.e.bias1) bias1 = p.e.bias1[ncl[0]];
    const bool has_res = EPI == 1 + EPI_DENSE && p.e.residual;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float res[4][NJ];
            if (has_res) {
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const int tok = min(m_wg + 32 * i + 8 * g + 4 * h + u, M - 1);
                        res[u][j] = p.e.residual[(size_t)tok * p.e.ldo + ncl[j]];
                    }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int t = 32 * i + 8 * g + 4 * h + u;
                const int tok = m_wg + t;
                if (tok >= M) continue;
                const double os0 = s_os0[t];
                const int xs = s_xs[t];
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    if (!ncol[j]) continue;
                    const int n = (nb0 + j) * 32 + l32;
                    const int raw0 = acc[0][i][j][4 * g + u];
                    if (EPI == 0) {
                        __builtin_nontemporal_store((float)((double)(raw0 - xs) * os0),
                                                    &p.e.out[(size_t)tok * p.e.ldo + n]);
                    } else {
                        const int raw1 = NMAT == 2 ? acc[NMAT - 1][i][j][4 * g + u] : raw0;
                        epilogue_store_pre<EPI - 1>(p.e, tok, n, raw0, raw1, os0, NMAT == 2 ? s_os1[t] : 0.0,
                                                    xs, bias0[j], bias1, has_res ? res[u][j] : 0.0f);
                    }
                }
            }
        }
}

// Tile height and split of a launch (measured on MI355X at both BitNet-2B FFN
// shapes, M = 65 .. 16384): 128-token tiles win once the grid has at least
// kTile128MinTiles of them (M = 16384: 2.1 vs 1.8 POPS at K = 2560, 2.5 vs
// 2.1 at K = 6912; M = 4096: 64-token tiles by up to 15 %).  Splitting
// K pays only while few tiles exist and every range keeps a long K loop: with
// at most kSplitMaxTiles tiles, about kSplitTarget workgroups in all, at least
// kMinSplitKtiles K tiles per range, at most kMaxSplit ranges.
constexpr int kTile128MinTiles = 1024;
// Half-width tiles (64 tokens x 128 weight rows, one workgroup of four waves
// each owning one 32-row block) on one matrix when the full-width 64-token
// grid has fewer tiles than the chip has CUs: twice the workgroups, so the
// CUs that would sit idle or run one wave per SIMD run two (measured at
// K = 2560 / 6912: M = 128 up 10.6 -> 7.6 us, down 12.4 -> 9.3; M = 256
// 10.6 -> 7.9 / 13.4 -> 10.6; M = 512 down 16.6 -> 15.4, up unchanged;
// M = 1024 up 21.7 -> 22.8, so that grid keeps full-width tiles).
constexpr int kHalfWidthMaxTiles = 256;
constexpr int kSplitMaxTilesPlan = 96;
constexpr int kSplitTarget = 240;
constexpr int kMinSplitKtiles = 6;
constexpr int kMaxSplit = 4;

struct GemmPlan {
    int mi, ksplit, sps, nj;
};

static GemmPlan plan_gemm(int m, int ntiles, int ktiles, int nmat, int device) {
    const int ngroups = ceil_div(ntiles, 16 / nmat);
    // LOOM_AMD_GEMM_TILE=128|64, LOOM_AMD_GEMM_SPLIT=n and LOOM_AMD_GEMM_NJ=1|2
    // override the choice (tuning and tests)
    const int force_tile = tune_int("LOOM_AMD_GEMM_TILE", 0);
    const int force_split = tune_int("LOOM_AMD_GEMM_SPLIT", 0);
    const int force_nj = tune_int("LOOM_AMD_GEMM_NJ", 0);
    if (force_tile == 128) return GemmPlan{4, 1, ktiles, 2 / nmat};
    // large grids take 128-token tiles (never split)
    if (force_tile != 64 && force_split == 0 && force_nj == 0 && ceil_div(m, 128) * ngroups >= kTile128MinTiles)
        return GemmPlan{4, 1, ktiles, 2 / nmat};
    // one matrix on a grid of fewer full-width tiles than CUs: half-width
    // tiles (128 weight rows, one 32-row block per wave)
    int nj = 2 / nmat;
    if (nmat == 1 && (force_nj == 1 || (force_nj == 0 && ceil_div(m, 64) * ngroups < kHalfWidthMaxTiles))) nj = 1;
    const int tiles = ceil_div(m, 64) * (nj == 1 && nmat == 1 ? ceil_div(ntiles, 8) : ngroups);
    int want = 1;
    if (force_split > 0) {
        want = force_split;
    } else if (tiles <= kSplitMaxTilesPlan) {
        want = ceil_div(kSplitTarget, tiles);
        if (want > ktiles / kMinSplitKtiles) want = ktiles / kMinSplitKtiles;
        if (want > kMaxSplit) want = kMaxSplit;
        if (want < 1) want = 1;
    }
    int sps = ceil_div(ktiles, want);
    if (sps > ktiles) sps = ktiles;
    int ks = ceil_div(ktiles, sps);
    const SplitWs ws = split_ws(device);
    if (ks > 1 && (!ws.part || tiles > kSplitTiles || tiles * ks > kSplitSlots)) ks = 1;
    return GemmPlan{2, ks, ks > 1 ? sps : ktiles, nj};
}

template <int NMAT, int EPI, int MI, int NJ>
static hipError_t launch_gemm_tile(const MatArgs& p, const GemmPlan& pl, int device, hipStream_t s) {
    GemmGrid gg;
    gg.mtiles = ceil_div(p.e.m, 32 * MI);
    gg.ngroups = ceil_div(p.ntiles, 8 * NJ);  // 16-row tiles per workgroup: 4 waves x NJ 32-row blocks
    gg.ksplit = pl.ksplit;
    gg.sps = pl.sps;
    gg.group = tune_int("LOOM_AMD_GEMM_GROUP", 8);
    const SplitWs ws = pl.ksplit > 1 ? split_ws(device) : SplitWs{};
    gg.part = ws.part;
    gg.ctr = ws.ctr;
    const int total = gg.mtiles * gg.ngroups * gg.ksplit;
    const int grid = ceil_div(total, kXcds) * kXcds;
    hipLaunchKernelGGL((gemm_lds_kernel<NMAT, EPI, MI, NJ>), dim3(grid), dim3(256), 0, s, p, gg);
    return hipGetLastError();
}

template <int NMAT, int EPI>
static hipError_t launch_gemm_planned(const MatArgs& p, int device, hipStream_t s) {
    const GemmPlan pl = plan_gemm(p.e.m, p.ntiles, p.ktiles, NMAT, device);
    if (pl.mi == 4) return launch_gemm_tile<NMAT, EPI, 4, 2 / NMAT>(p, pl, device, s);
    if constexpr (NMAT == 1) {
        if (pl.nj == 1) return launch_gemm_tile<1, EPI, 2, 1>(p, pl, device, s);
    }
    return launch_gemm_tile<NMAT, EPI, 2, 2 / NMAT>(p, pl, device, s);
}

static bool plain_dense(const EpiDev& e) {
    return e.kind == EPI_DENSE && !e.bias0 && !e.residual && !e.post && !e.acc0;
}

hipError_t launch_gemm(const MatArgs& p, bool two, int device, hipStream_t s) {
    if (two) return launch_gemm_planned<2, 1 + EPI_SWIGLU>(p, device, s);
    if (plain_dense(p.e)) return launch_gemm_planned<1, 0>(p, device, s);
    if (p.e.kind == EPI_ACC) return launch_gemm_planned<1, 1 + EPI_ACC>(p, device, s);
    return launch_gemm_planned<1, 1 + EPI_DENSE>(p, device, s);
}

}  // namespace lamd
