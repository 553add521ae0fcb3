// Shared device code for the gfx950 FlashAttention kernels: element types, MFMA
// wrappers, LDS swizzles, sequence bookkeeping and block-granular tile ranges.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mykfa.h"

namespace mykfa {

typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr float kNegFloor = -1e30f;  // finite row-max floor (flash_attn.py:136-137)
// A running softmax max is only raised when a tile exceeds it by more than this (log2 units),
// bounding unnormalized probabilities by 2^8.
constexpr float kRescaleSlack = 8.0f;

// ---- element types -------------------------------------------------------------------

struct BF16 {
    static constexpr int code = MYKFA_BF16;
    __device__ static inline uint16_t from_float(float x) {
        __bf16 b = (__bf16)x;  // round to nearest even (v_cvt_pk_bf16_f32)
        return __builtin_bit_cast(uint16_t, b);
    }
    __device__ static inline float to_float(uint16_t x) {
        return __uint_as_float(((uint32_t)x) << 16);
    }
    // Two floats rounded to nearest even and packed in one v_cvt_pk_bf16_f32.
    __device__ static inline uint32_t pack2(float a, float b) {
        // A 2-vector conversion: two scalar casts compile to two half-empty conversions and a
        // v_perm_b32 to merge them.
        const f32x2 v = {a, b};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    }
    // c + x.lo + x.hi for a packed pair, in fp32 (v_dot2c_f32_bf16 against (1, 1)).
    __device__ static inline float sum2(uint32_t x, float c) {
        const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), ones, c, false);
    }
    // C(32x32) += A(32x16) * B(16x32); lane l holds A[l%32][8(l/32)+i], B[8(l/32)+i][l%32].
    __device__ static inline f32x16 mfma32(s16x8 a, s16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    // C(16x16) += A(16x32) * B(32x16); lane l holds A[l%16][8(l/16)+i], B[8(l/16)+i][l%16].
    __device__ static inline f32x4 mfma16(s16x8 a, s16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};

struct FP16 {
    static constexpr int code = MYKFA_FP16;
    __device__ static inline uint16_t from_float(float x) {
        _Float16 h = (_Float16)x;
        return __builtin_bit_cast(uint16_t, h);
    }
    __device__ static inline float to_float(uint16_t x) {
        return (float)__builtin_bit_cast(_Float16, x);
    }
    __device__ static inline uint32_t pack2(float a, float b) {
        const f32x2 v = {a, b};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
    }
    __device__ static inline float sum2(uint32_t x, float c) {
        const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), ones, c, false);
    }
    __device__ static inline f32x16 mfma32(s16x8 a, s16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    __device__ static inline f32x4 mfma16(s16x8 a, s16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};

// ---- small helpers ---------------------------------------------------------------------

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// v_permlane32_swap with both operands x returns, in every lane l, the pair
// (x[l % 32], x[32 + l % 32]): the values of the two lanes that share a query column of a
// 32x32 MFMA tile. Combining the pair reduces over that column's two lane groups.
__device__ inline float max_halves(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float sum_halves(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// A fresh scalar copy of a wave-uniform value. Kernel arguments arrive as wide scalar-load
// tuples; a loop that keeps one element live keeps (and, under pressure, spills) the whole
// tuple, while an opaque copy lets the tuple die.
__device__ inline int sgpr_copy(int x) {
    x = __builtin_amdgcn_readfirstlane(x);
    asm volatile("" : "+s"(x));
    return x;
}
__device__ inline float sgpr_copy(float x) { return __int_as_float(sgpr_copy(__float_as_int(x))); }
__device__ inline int64_t sgpr_copy(int64_t x) {
    const uint32_t lo = (uint32_t)sgpr_copy((int)(uint32_t)x);
    const uint32_t hi = (uint32_t)sgpr_copy((int)(uint32_t)((uint64_t)x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// 16-byte and 8-byte global accesses.
__device__ inline s16x8 ld16(const uint16_t* p) { return *reinterpret_cast<const s16x8*>(p); }
// The same with the non-temporal (streaming) hint, for tensors a kernel reads exactly once.
__device__ inline s16x8 ld16_stream(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const s16x8*>(p));
}
__device__ inline void st16(uint16_t* p, s16x8 v) { *reinterpret_cast<s16x8*>(p) = v; }

// ds_read_b64_tr_b16: within each group of 16 lanes, lane j receives, for i = 0..3, element
// (j % 4) of the 4-element vector addressed by lane (4 i + j / 4) of its group. When lane
// s = 4 i + b of the group points at row (r0 + i), column (c0 + 4 b) of a row-major matrix,
// lane j receives rows r0..r0+3 of column c0 + j: a transposed 4x16 read.
__device__ inline s16x4 ds_read_tr(const uint16_t* lds_ptr) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr));
}

__device__ inline s16x8 cat4(s16x4 a, s16x4 b) {
    return s16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// ---- LDS layout -----------------------------------------------------------------------
// Tiles of ROWS x D 16-bit elements live row-major in LDS as 16-byte chunks; chunk c of row
// r is stored at chunk position c ^ swz(r). gfx950's LDS serves 64 banks x 4 bytes (256 bytes)
// per cycle: a 16-byte-per-lane read is served 16 lanes at a time and a transpose read
// (8 bytes per lane) 32 lanes at a time, so each such lane group must cover all 256 bytes of
// bank space once. The two patterns of the kernels:
//  - row-operand read: 16 lanes read rows 0..15 of an aligned 16-row group (perm32 order) at
//    one logical chunk c;
//  - transpose read: 32 lanes read 4 consecutive rows r0..r0+3 (r0 = 0 mod 4) at 4 aligned
//    logical chunks 4b..4b+3 (two 8-byte halves each).
// Per head_dim (16-byte slots of bank space: 16 per 256 bytes):
//  - D >= 128 (a row spans >= 256 bytes): swz = 4 (r mod 4) + (r / 4 mod 4) is a bijection of
//    the 16 rows (row read), and its top two bits, r mod 4, differ across any 4 consecutive
//    rows, so the 4 x 4 (row, chunk) slots of a transpose read are distinct;
//  - D = 64 (two rows per 256 bytes; slot = 8 (r mod 2) + chunk): swz = 4 (r / 2 mod 2) +
//    (r / 4 mod 4) is a bijection on the 8 rows of each parity, and its top bit differs
//    between rows r and r + 2;
//  - D = 32 (four rows per 256 bytes): swz = r / 4 mod 4; D = 16 (eight rows): swz = r / 8 mod 2.
// Measured with SQ_LDS_BANK_CONFLICT: 0 conflict cycles for both patterns (the previous
// layout, built for 32 banks, took one conflict cycle per active cycle).
template <int D>
__device__ inline int lds_swz(int row) {
    if constexpr (D >= 128) return ((row & 3) << 2) | ((row >> 2) & 3);
    else if constexpr (D == 64) return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
    else if constexpr (D == 32) return (row >> 2) & 3;
    else return (row >> 3) & 1;
}
template <int D>
__device__ inline int lds_off(int row, int col) {  // element offset of (row, col)
    return row * D + ((((col >> 3) ^ lds_swz<D>(row))) << 3) + (col & 7);
}

// Row permutation used when a 32-row tile is the A operand of a 32x32x16 MFMA whose output
// then feeds another MFMA as its k-operand: swapping rows 4-7 with 8-11 (in each 16) makes
// output register r of lane group g hold row 16 (r / 8) + 8 g + r % 8, i.e. each lane
// group holds 8 consecutive rows per 16, the k-slot order of the next MFMA.
__device__ inline int perm32(int rho) { return (rho & ~12) | ((rho & 4) << 1) | ((rho & 8) >> 1); }
// Tile row held by output register r (0..15) of lane group g after the permuted load.
__device__ inline int out_row32(int r, int g) { return 16 * (r >> 3) + 8 * g + (r & 7); }

// ---- waits and barriers ---------------------------------------------------------------------
// s_waitcnt immediates (gfx9 layout: vmcnt[3:0] + [15:14], expcnt[6:4], lgkmcnt[11:8]).
template <int N>
__device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ inline void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }
// Workgroup barrier without the release/acquire fences of __syncthreads(), whose release
// half would drain every in-flight load (vmcnt(0)) and defeat the asynchronous tile ring.
// Callers order LDS themselves: all ds_read results are consumed before the barrier and
// DMA tile loads are waited for with wait_vmcnt<>.
__device__ inline void barrier_lds() {
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
}

// ---- asynchronous tile ring (buffer_load ... lds) ---------------------------------------
// Rows [n0, n0 + ROWS) x D of NT tensors (16-bit, row stride in elements) are fetched straight
// into a swizzled LDS tile by buffer loads with the LDS destination: lane l of a load writes
// 16 bytes at LDS base + 16 l, so each lane fetches the global chunk whose swizzled LDS slot is
// that position. The buffer resource covers exactly the sequence's valid rows, so rows at or
// beyond the length read as zero without touching memory. Each wave issues LOADS loads per
// tile; completion is tracked per wave with wait_vmcnt and made workgroup-visible by a barrier.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer descriptor over [base, base + bytes): loads at offsets >= bytes return zero.
__device__ inline i32x4 buffer_rsrc(const void* base, int64_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    // Wave-uniform by construction; readfirstlane places it in scalar registers as the buffer
    // instructions require.
    i32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)(a & 0xffffffffu));
    r[1] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)((a >> 32) & 0xffffu));  // stride 0
    r[2] = __builtin_amdgcn_readfirstlane((int32_t)(bytes > 0x7fffffff ? 0x7fffffff : bytes));
    r[3] = 0x00020000;
    return r;
}
// The same from a wave-uniform address and a byte range already known to fit 31 bits.
__device__ inline i32x4 buffer_rsrc32(uint64_t a, int bytes) {
    i32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)(a & 0xffffffffu));
    r[1] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)((a >> 32) & 0xffffu));  // stride 0
    r[2] = __builtin_amdgcn_readfirstlane(bytes);
    r[3] = 0x00020000;
    return r;
}
// Descriptor over the valid rows [0, rows) of a (rows, D) 16-bit tensor with row stride tstride.
__device__ inline i32x4 rows_rsrc(const uint16_t* base, int rows, int64_t tstride, int D) {
    return buffer_rsrc(base, rows > 0 ? ((int64_t)(rows - 1) * tstride + D) * 2 : 0);
}
// LDS byte address of a pointer into __shared__ memory.
__device__ inline uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(p);
}
// buffer_load ... lds: every active lane fetches 16 (or 4) bytes at voff and the wave writes
// them to LDS at lds_base + 16 (4) x lane. Issued through inline asm so the compiler does not
// track these LDS writes: it would otherwise drain the load counter before every LDS
// transpose read it cannot disambiguate. Completion is awaited explicitly (wait_vmcnt), and
// no compiler-generated code in these kernels keeps a value in m0 across them.
__device__ inline void dma16(i32x4 rsrc, uint32_t lds_base, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}
// The same with the non-temporal hint, for data read exactly once (streamed past the caches'
// reuse): the dS pass measured 199 -> 180 us with it.
__device__ inline void dma16_nt(i32x4 rsrc, uint32_t lds_base, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}
__device__ inline void dma4(i32x4 rsrc, uint32_t lds_base, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

template <int D, int ROWS, int NT, int NW>
struct TileRing {
    static constexpr int CPR = D / 8;
    static constexpr int LOADS_PER_TENSOR = ROWS * CPR / 64;  // 64-lane loads per tensor tile
    static constexpr int LOADS = NT * LOADS_PER_TENSOR / NW;  // per wave per tile
    static_assert((ROWS * CPR) % 64 == 0, "tile must be whole 64-lane loads");
    static_assert((NT * LOADS_PER_TENSOR) % NW == 0, "loads must split evenly over the waves");

    // tiles[t] = LDS tile of tensor t (ROWS * D elements); rsrc[t] / tstride_bytes[t] its source.
    __device__ static inline void issue(const i32x4* rsrc, const int* tstride_bytes, uint16_t* const* tiles,
                                        int n0, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            const int instr = wave * LOADS + j;
            const int t = instr / LOADS_PER_TENSOR, within = instr % LOADS_PER_TENSOR;
            const int p = within * 64 + lane;
            const int row = p / CPR, phys = p % CPR;
            const int logical = phys ^ lds_swz<D>(row);
            const unsigned voff = (unsigned)((n0 + row) * tstride_bytes[t] + logical * 16);
            dma16(rsrc[t], lds_addr(tiles[t] + within * 512), voff);
        }
    }
};

// Wait until the tile issued `ahead` tiles before the newest one has landed (this wave's part).
template <int LOADS, int STAGES>
__device__ inline void ring_wait(int tiles_after) {
    // tiles_after = tiles issued after the awaited one, 0 .. STAGES - 2 (the load counter
    // holds at most 63 outstanding loads).
    static_assert((STAGES - 2) * LOADS <= 63, "ring deeper than the load counter");
    if constexpr (STAGES >= 6) {
        if (tiles_after >= 4) return wait_vmcnt<4 * LOADS>();
    }
    if constexpr (STAGES >= 5) {
        if (tiles_after >= 3) return wait_vmcnt<3 * LOADS>();
    }
    if constexpr (STAGES >= 4) {
        if (tiles_after >= 2) return wait_vmcnt<2 * LOADS>();
    }
    if constexpr (STAGES >= 3) {
        if (tiles_after >= 1) return wait_vmcnt<LOADS>();
    }
    wait_vmcnt<0>();
}

// ---- XCD-aware workgroup order ------------------------------------------------------------
// MI355X has 8 XCDs, each with its own L2; the dispatcher deals workgroup i to XCD i % 8. The
// launchers pad a 1-D grid to a multiple of 8 * kXcdChunk and each workgroup maps its id to a
// logical block so that every run of kXcdChunk consecutive logical blocks (neighbouring
// query / key blocks of one head, which read the same K/V or Q/dO tiles) executes on one XCD
// and shares its L2. Logical ids >= n (padding) exit at once.
constexpr int kXcds = 8;
constexpr int kXcdChunk = 4;
__host__ __device__ inline int xcd_grid(int n) {
    const int q = kXcds * kXcdChunk;
    return (n + q - 1) / q * q;
}
__device__ inline int xcd_logical(int pid) {
    const int xcd = pid % kXcds, slot = pid / kXcds;
    return ((slot / kXcdChunk) * kXcds + xcd) * kXcdChunk + slot % kXcdChunk;
}

// Block order for grids whose per-block work is skewed (causal rows or keys). A logical id
// decodes block-rank-slowest: ranks r*kXcdChunk .. r*kXcdChunk + kXcdChunk - 1 of every
// (group, sequence) are dispatched before the next run of ranks, so the longest blocks of ALL
// heads and sequences start first (longest-processing-time order; a doc-major order leaves
// the long causal blocks of the last sequences for the tail) while each run of kXcdChunk
// consecutive blocks of one (group, sequence) still executes on one XCD. Ranks >= the block
// count (padding) are for the caller to skip.
//
// Run j of a (group, sequence) pair is run index R = j * P + pair, which executes on XCD R % 8.
// For packed (varlen) batches, whose sequences differ in length and so in work, from 8 pairs
// on P is padded (idle pairs exit at once) to P = 4 (mod 8), so that the runs of
// a pair alternate between two XCDs, pair % 8 and pair % 8 + 4 (below 8 pairs P stays as it
// is: the pairs then rotate through 8, 4 or 2 XCDs each and still cover all). With P a multiple of 8
// every run of a pair lands on one XCD: the XCDs holding the longest sequences then carry most
// of the work while the others idle (measured: 30% more work on half of the XCDs for 8
// sequences x 4 KV heads). Spreading a pair over all eight XCDs (P odd) balances the work but
// costs each XCD's L2 the pair's tiles eight times over, which measured slower; two XCDs per
// pair, in runs of kXcdChunk = 4 ranks, measured best (5-8% on a skewed varlen batch, within
// noise on long ones; shorter runs lost up to a quarter to L2 misses). Dense batches, whose
// pairs all carry the same work, keep P unpadded: every pair on one XCD (2-5% faster there).
struct BlockCoord {
    int rank, group, seq;
};
__host__ __device__ inline int coord_pairs(int groups, int seqs, bool varlen) {
    const int p = groups * seqs;
    return (!varlen || p < 8) ? p : p + (12 - p % 8) % 8;
}
__device__ inline BlockCoord block_coord(int logical, int groups, int seqs, bool varlen) {
    const int lo = logical % kXcdChunk, rest = logical / kXcdChunk;
    const int P = coord_pairs(groups, seqs, varlen);
    const int j = rest / P, pair = rest % P;
    BlockCoord c;
    c.group = pair % groups;
    c.seq = pair / groups;
    c.rank = pair < groups * seqs ? j * kXcdChunk + lo : 0x3fffffff;  // idle pair: no block
    return c;
}
inline long long block_grid_size(int nblk, int groups, int seqs, bool varlen) {
    return (long long)((nblk + kXcdChunk - 1) / kXcdChunk) * kXcdChunk * coord_pairs(groups, seqs, varlen);
}

// ---- sequences --------------------------------------------------------------------------

struct SeqInfo {
    int64_t tok0;  // first token of the sequence in the (packed) tensor
    int64_t row0;  // first row in the (heads, rows) lse/delta buffers
    int len;
};

// flash_attn.py:39-55 (_seq_info).
__device__ inline SeqInfo seq_info(int b, const int32_t* cu, const int32_t* seqused, int seqlen,
                                   bool use_seqused) {
    SeqInfo s;
    if (cu != nullptr) {
        int start = cu[b];
        s.len = cu[b + 1] - start;
        s.tok0 = start;
        s.row0 = start;
    } else {
        s.tok0 = 0;
        s.row0 = (int64_t)b * seqlen;
        int len = seqlen;
        if (use_seqused && seqused != nullptr) {  // clamp: never read beyond the cache capacity
            len = seqused[b];
            len = len < 0 ? 0 : (len > seqlen ? seqlen : len);
        }
        s.len = len;
    }
    return s;
}

// Block ranges, flash_attn.py:58-68 (_block_ranges). For "self" indices [s0, s0 + BS),
// each seeing "other" indices t with lo_off <= t - s <= hi_off and 0 <= t < t_len, the
// BT-aligned range [lo, hi) of t to visit, split as [lo, mid_lo) masked,
// [mid_lo, mid_hi) unmasked for every s, [mid_hi, hi) masked.
struct Ranges {
    int lo, mid_lo, mid_hi, hi;
};
__host__ __device__ inline Ranges block_ranges(int s0, int BS, int lo_off, int hi_off, int t_len, int BT) {
    Ranges r;
    int a = s0 + lo_off;
    r.lo = (a > 0 ? a : 0) / BT * BT;
    int h = s0 + BS + hi_off;
    h = h < t_len ? h : t_len;
    r.hi = h > r.lo ? h : r.lo;
    int m = s0 + BS - 1 + lo_off;
    m = m > r.lo ? m : r.lo;
    int ml = (m + BT - 1) / BT * BT;  // m >= lo >= 0
    r.mid_lo = ml < r.hi ? ml : r.hi;
    int mh = s0 + hi_off + 1;
    mh = mh < t_len ? mh : t_len;
    mh = mh > 0 ? mh : 0;
    mh = mh / BT * BT;
    r.mid_hi = mh > r.mid_lo ? mh : r.mid_lo;
    return r;
}

// Offsets of windowed causal masking: query i sees key j iff lo_off <= j - i <= hi_off.
__host__ __device__ inline int band_lo(int k_len, int q_len, int wl) { return k_len - q_len - wl; }
__host__ __device__ inline int band_hi(int k_len, int q_len, int wr) {
    // wr may be 2^30: keep the sum within int32
    long long v = (long long)k_len - q_len + wr;
    return v > (1 << 30) ? (1 << 30) : (int)v;
}

// Band mask of the 16 output registers of a 32x32 MFMA tile, without per-element compares.
// Register r = 8 h + i (h = 0, 1; i = 0..7) holds index base + 16 h + i of the masked
// dimension, and the lane's visible indices form one inclusive range [lo, hi] (empty when
// hi < lo). Each run of 8 gets an 8-bit mask from two clamps; an element is kept by a bit
// select with the sign-extended mask bit (0 or -1): masked elements become the float whose
// bits are `fill` (+0 by default; 0xff800000 is -inf) whatever they held. Per-element compares
// would each produce a 64-bit condition mask in scalar registers; unrolled over 16 elements
// those exhaust the scalar register file and spill.
__device__ inline void mask_runs16(float* v, int base, int lo, int hi, unsigned fill = 0u) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int r0 = base + 16 * h;
        const int a = min(max(lo - r0, 0), 8);
        const int b = min(max(hi - r0 + 1, 0), 8);
        const unsigned bits = ((1u << b) - 1u) & ~((1u << a) - 1u);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned keep = (unsigned)((int)(bits << (31 - i)) >> 31);
            v[8 * h + i] = __uint_as_float((__float_as_uint(v[8 * h + i]) & keep) | (fill & ~keep));
        }
    }
}

}  // namespace mykfa
