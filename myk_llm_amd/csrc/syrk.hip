// Batched symmetric rank-K product of Muon's Newton-Schulz iteration (replaces
// _batched_syrk_kernel, ops/muon.py:28-104):
//   Out[b] = alpha * X[b] X[b]^T + beta * Bias[b],   X (batch, M, K) bf16, Out (batch, M, M) bf16.
// Only the lower-triangular 128 x 128 output tiles are computed; an off-diagonal tile is also
// stored transposed into the upper triangle (Bias is read at the computed positions only, so a
// symmetric Bias gives the full symmetric result, as in the reference).
//
// One workgroup = one output tile, 4 waves in 2 x 2, each wave a 64 x 64 quarter as 2 x 2
// blocks of 32x32x16 bf16 MFMA with fp32 accumulation. K advances 64 columns per stage through
// a 2-stage asynchronous LDS ring (buffer_load ... lds straight into swizzled tiles; one stage
// loads while the other is consumed): a stage holds the 128 x 64 row panels of X at the tile's
// row block (A) and column block (B). Both MFMA operands are row reads of those panels (X X^T:
// the B operand of column n is row n of X), taken in the permuted row order under which a
// 16-byte row read touches every LDS bank once; the permutation is undone when the tile is
// stored. 64 KB of LDS keeps two workgroups resident per CU (measured: a third 32 KB stage,
// one workgroup per CU, is 1.8x slower at 9 x 1024 x 4096; 32-column stages 1.2x slower).
#include "common.h"
#include "kernels.h"

namespace mykfa {
namespace {

constexpr int kBM = 128;                             // output tile rows = columns
constexpr int kBK = 64;                              // K columns per stage
constexpr int kStages = 2;
constexpr int kNW = 4;                               // waves per workgroup (2 x 2)
constexpr int kCPR = kBK / 8;                        // 16-byte chunks per panel row
constexpr int kLoadsPerPanel = kBM * kCPR / 64;      // 64-lane loads per 128 x kBK panel
constexpr int kLoads = 2 * kLoadsPerPanel / kNW;     // loads per wave per stage (A and B panels)
static_assert((2 * kLoadsPerPanel) % kNW == 0, "panel loads split evenly over the waves");

// Lower-triangular tile index -> (tile row, tile column), column <= row.
__device__ inline void tile_coord(int pid, int& tm, int& tn) {
    int r = (int)((sqrtf(8.0f * (float)pid + 1.0f) - 1.0f) * 0.5f);
    while (r * (r + 1) / 2 > pid) --r;
    while ((r + 1) * (r + 2) / 2 <= pid) ++r;
    tm = r;
    tn = pid - r * (r + 1) / 2;
}

// A operand (32 rows x 16 k) of a panel at rows rbase + perm32(l32), k-step kk.
__device__ inline s16x8 panel_op(const uint16_t* panel, int rbase, int l32, int g, int kk) {
    const int row = rbase + perm32(l32);
    return *reinterpret_cast<const s16x8*>(panel + row * kBK + (((2 * kk + g) ^ lds_swz<kBK>(row)) << 3));
}

__device__ inline float bias_at(const mykfa_syrk_params& p, int bidx, int i, int j) {
    const uint16_t* bp = static_cast<const uint16_t*>(p.bias) + (int64_t)bidx * p.bias_batch_stride;
    return BF16::to_float(bp[(int64_t)i * p.bias_row_stride + j]);
}

// Workgroup id -> (matrix, tile). The dispatcher deals workgroup i to XCD i % 8; XCD x is
// given the contiguous run [x * per_xcd, (x + 1) * per_xcd) of the matrix-major unit list, so
// the tiles of one matrix (8 tiles per row panel of X) share one XCD's L2 instead of each XCD
// fetching nearly every panel of every matrix. Ids past the last unit do nothing.
__device__ inline bool syrk_unit(int pid, int per_xcd, int tiles_per_matrix, int units, int& bidx, int& tile) {
    const int unit = (pid % kXcds) * per_xcd + pid / kXcds;
    bidx = unit / tiles_per_matrix;
    tile = unit - bidx * tiles_per_matrix;
    return unit < units;
}

__global__ __launch_bounds__(kNW * 64) void syrk_kernel(mykfa_syrk_params p, int per_xcd, int tiles_per_matrix) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[kStages][2][kBM * kBK];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, l32 = lane & 31, g = lane >> 5;
    int bidx, tile;
    if (!syrk_unit(blockIdx.x, per_xcd, tiles_per_matrix, p.batch * tiles_per_matrix, bidx, tile)) return;
    int tm, tn;
    tile_coord(tile, tm, tn);
    const int m0 = tm * kBM, n0 = tn * kBM;

    // Panel sources: rows [m0, m0 + 128) and [n0, n0 + 128) of X[bidx]; the descriptors cover
    // only the valid rows, so rows at or beyond M read as zero.
    const uint16_t* xb = static_cast<const uint16_t*>(p.x) + (int64_t)bidx * p.x_batch_stride;
    const int64_t xrs = p.x_row_stride;
    const uint64_t src0 = reinterpret_cast<uint64_t>(xb + (int64_t)m0 * xrs);
    const uint64_t src1 = reinterpret_cast<uint64_t>(xb + (int64_t)n0 * xrs);
    const int rows0 = min(p.m - m0, kBM), rows1 = min(p.m - n0, kBM);
    const int bytes0 = (int)(((int64_t)(rows0 - 1) * xrs + p.k) * 2);
    const int bytes1 = (int)(((int64_t)(rows1 - 1) * xrs + p.k) * 2);
    // Loop-invariant lane offsets: load j of this wave fills 64 chunks of panel t.
    unsigned voff[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int within = (wave * kLoads + j) % kLoadsPerPanel;
        const int pch = within * 64 + lane;
        const int row = pch / kCPR, phys = pch % kCPR;
        voff[j] = (unsigned)(row * (int)(xrs * 2) + ((phys ^ lds_swz<kBK>(row)) << 4));
    }
    const uint32_t lds0 = lds_addr(&smem[0][0][0]);
    const int nk = p.k / kBK;
    auto issue = [&](int kt) {
        const uint32_t stage = lds0 + (uint32_t)((kt % kStages) * 2 * kBM * kBK * 2);
        const int kb = kt * kBK * 2;  // byte offset of the stage's first column
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int instr = wave * kLoads + j;
            const int t = instr / kLoadsPerPanel, within = instr % kLoadsPerPanel;
            const i32x4 rsrc = t == 0 ? buffer_rsrc32(src0 + kb, bytes0 - kb) : buffer_rsrc32(src1 + kb, bytes1 - kb);
            dma16(rsrc, stage + (uint32_t)((t * kBM * kBK + within * 512) * 2), voff[j]);
        }
    };
#pragma unroll
    for (int t = 0; t < kStages - 1; ++t)
        if (t < nk) issue(t);

    f32x16 acc[2][2];
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[bi][bj][r] = 0.f;
    const int wm = wave >> 1, wn = wave & 1;

    for (int kt = 0; kt < nk; ++kt) {
        const int after = nk - 1 - kt < kStages - 2 ? nk - 1 - kt : kStages - 2;
        ring_wait<kLoads, kStages>(after);
        barrier_lds();  // stage kt landed for every wave; stage kt - 1 is free again
        if (kt + kStages - 1 < nk) issue(kt + kStages - 1);
        const uint16_t* As = smem[kt % kStages][0];
        const uint16_t* Bs = smem[kt % kStages][1];
        // Every operand of the stage is read before its products: left to itself the compiler
        // reads, waits and multiplies one k-step at a time, exposing the LDS latency per step.
        s16x8 av[kBK / 16][2], bv[kBK / 16][2];
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            av[kk][0] = panel_op(As, wm * 64, l32, g, kk);
            av[kk][1] = panel_op(As, wm * 64 + 32, l32, g, kk);
            bv[kk][0] = panel_op(Bs, wn * 64, l32, g, kk);
            bv[kk][1] = panel_op(Bs, wn * 64 + 32, l32, g, kk);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            acc[0][0] = BF16::mfma32(av[kk][0], bv[kk][0], acc[0][0]);
            acc[0][1] = BF16::mfma32(av[kk][0], bv[kk][1], acc[0][1]);
            acc[1][0] = BF16::mfma32(av[kk][1], bv[kk][0], acc[1][0]);
            acc[1][1] = BF16::mfma32(av[kk][1], bv[kk][1], acc[1][1]);
        }
    }

    // Epilogue: register r of lane (g, l32) holds C[perm32(8 (r / 4) + 4 g + r % 4)][perm32(l32)]
    // of its 32 x 32 block (both operands were read in perm32 order); perm32 keeps bits 0-1, so
    // registers 4q..4q+3 are 4 consecutive rows -- 4 consecutive columns of the mirrored store.
    uint16_t* ob = static_cast<uint16_t*>(p.out) + (int64_t)bidx * p.out_batch_stride;
    const int64_t ors = p.out_row_stride;
    const bool mirror = tm != tn;
    const bool has_bias = p.bias != nullptr;
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
            const int gj = n0 + wn * 64 + 32 * bj + perm32(l32);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int gi0 = m0 + wm * 64 + 32 * bi + perm32(8 * q + 4 * g);
                uint16_t o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int gi = gi0 + e;
                    float v = acc[bi][bj][4 * q + e] * p.alpha;
                    if (has_bias && gi < p.m && gj < p.m) v += p.beta * bias_at(p, bidx, gi, gj);
                    o[e] = BF16::from_float(v);
                    if (gi < p.m && gj < p.m) ob[(int64_t)gi * ors + gj] = o[e];
                }
                if (mirror && gj < p.m) {
                    uint16_t* dst = ob + (int64_t)gj * ors + gi0;
                    if (gi0 + 3 < p.m) {
                        u32x2 w = {(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
                        *reinterpret_cast<u32x2*>(dst) = w;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (gi0 + e < p.m) dst[e] = o[e];
                    }
                }
            }
        }
}

}  // namespace

hipError_t launch_syrk(const mykfa_syrk_params& p, hipStream_t stream) {
    const long long tiles = (long long)(p.m + kBM - 1) / kBM;
    const long long per_matrix = tiles * (tiles + 1) / 2;
    const long long per_xcd = (per_matrix * p.batch + kXcds - 1) / kXcds;
    if (per_xcd * kXcds >= (1ll << 31)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(syrk_kernel, dim3((unsigned)(per_xcd * kXcds)), dim3(kNW * 64), 0, stream, p, (int)per_xcd,
                       (int)per_matrix);
    return hipGetLastError();
}

}  // namespace mykfa
