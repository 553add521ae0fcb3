// Prefill forward: O and base-2 LSE (replaces _fwd_kernel, flash_attn.py:106-154).
//
// Work decomposition. A workgroup is NW waves (4); every wave
// owns 32 query rows of one head. The workgroup's waves cover `hpw` query heads of ONE GQA
// group (hpw = gcd(group, NW)) times NW / hpw blocks of 32 consecutive tokens, so each K/V
// tile staged in LDS serves every query head of the group that the workgroup holds: K/V
// bytes are fetched once per group.
//
// Per 64-key tile, each wave computes S^T = K Q^T on 32x32x16 bf16 MFMA (K from LDS as the
// A operand, Q resident in registers as the B operand), so that the output lane of every
// score is its query and the registers are keys. The online softmax (row max on raw scores
// through a permlane32 swap, one FMA + exp2 per score, lazy rescaling of O) then produces
// P^T already in the k-operand layout of the next product O^T += V^T P^T, whose A operand
// (V^T) is read straight from the row-major V tile with the gfx950 LDS transpose read. K/V
// tiles arrive through an asynchronous LDS ring (buffer_load ... lds, STAGES - 1 tiles
// ahead) in an XOR-swizzled layout; one workgroup barrier per tile. Key tiles wholly outside
// a wave's causal/window band are skipped, and only tiles that cross the band edge evaluate
// the element mask (the 3-range split of flash_attn.py:140-145).
#include "common.h"
#include "kernels.h"

namespace mykfa {

namespace {

struct FwdArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    uint16_t* o;
    float* lse;
    int64_t qbs, qts, qhs, kbs, kts, khs, vbs, vts, vhs, obs, ots, ohs, lse_hs;
    const int32_t* cu_q;
    const int32_t* cu_k;
    const int32_t* seqused_k;
    int seqlen_q, seqlen_k;
    int wl, wr;
    float qk_scale;  // softmax_scale * log2(e)  (flash_attn.py:368)
    int group;       // num_heads / num_kv_heads
    int hpw;         // query heads per workgroup
    int gx, gy, gz;  // query blocks, sequences, head groups; decoded by block_coord
};

// Stage a BN x D tile (rows n0.., masked to < len) from global into a swizzled LDS tile.
template <int D, int BN, int NW, int STAGES, typename T>
__global__ __launch_bounds__(NW * 64) void fwd_kernel(FwdArgs a) {
    constexpr int KD = D / 16;            // k-steps of S^T = K Q^T
    constexpr int DB = (D + 31) / 32;     // 32-row blocks of O^T
    constexpr int NB = BN / 32;           // 32-key blocks per tile
    constexpr int KB = BN / 16;           // 16-key k-steps of O^T += V^T P^T
    using Ring = TileRing<D, BN, 2, NW>;  // K and V tiles
    __shared__ __attribute__((aligned(16))) uint16_t smem[STAGES][2][BN * D];

    const int tid = __builtin_amdgcn_workitem_id_x();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int l32 = lane & 31, g = lane >> 5;
    const int tpw = NW / a.hpw;
    // Longest causal rows first across all heads and sequences (flash_attn.py:115 orders
    // within one head only), XCD-grouped.
    const BlockCoord bc = block_coord(xcd_logical(__builtin_amdgcn_workgroup_id_x()), a.gz, a.gy, a.cu_q != nullptr);
    if (bc.rank >= a.gx) return;
    const int mblk = a.gx - 1 - bc.rank;
    const int h_first = bc.group * a.hpw;
    const int b = bc.seq;

    SeqInfo qs = seq_info(b, a.cu_q, nullptr, a.seqlen_q, false);
    const int tok_base = mblk * tpw * 32;
    if (tok_base >= qs.len) return;
    SeqInfo ks = seq_info(b, a.cu_k, a.seqused_k, a.seqlen_k, true);
    const int q_len = qs.len, k_len = ks.len;
    const int kvh = h_first / a.group;
    const int lo_off = band_lo(k_len, q_len, a.wl);
    const int hi_off = band_hi(k_len, q_len, a.wr);

    // Key range of the workgroup: union over its token blocks.
    int wg_lo = 1 << 30, wg_hi = 0;
    for (int tb = 0; tb < tpw; ++tb) {
        int s0 = tok_base + tb * 32;
        int bs = q_len - s0 < 32 ? q_len - s0 : 32;
        if (bs <= 0) continue;
        Ranges r = block_ranges(s0, bs, lo_off, hi_off, k_len, BN);
        if (r.hi > r.lo) {
            wg_lo = r.lo < wg_lo ? r.lo : wg_lo;
            wg_hi = r.hi > wg_hi ? r.hi : wg_hi;
        }
    }

    const int h = h_first + (wave % a.hpw);
    const int s0 = tok_base + (wave / a.hpw) * 32;
    const int bs = q_len - s0 < 32 ? q_len - s0 : 32;
    Ranges wr = {0, 0, 0, 0};
    if (bs > 0) wr = block_ranges(s0, bs, lo_off, hi_off, k_len, BN);

    const uint16_t* kbase = a.k + (int64_t)b * a.kbs + ks.tok0 * a.kts + (int64_t)kvh * a.khs;
    const uint16_t* vbase = a.v + (int64_t)b * a.vbs + ks.tok0 * a.vts + (int64_t)kvh * a.vhs;
    const i32x4 rsrc[2] = {rows_rsrc(kbase, k_len, a.kts, D), rows_rsrc(vbase, k_len, a.vts, D)};
    const int tstride[2] = {(int)(a.kts * 2), (int)(a.vts * 2)};

    const int ntiles = wg_hi > wg_lo ? (wg_hi - wg_lo + BN - 1) / BN : 0;
    auto issue = [&](int t) {
        uint16_t* tiles[2] = {smem[t % STAGES][0], smem[t % STAGES][1]};
        Ring::issue(rsrc, tstride, tiles, wg_lo + t * BN, wave, lane);
    };
    // The ring's first tiles go out before the Q loads, so the two latencies overlap.
#pragma unroll
    for (int t = 0; t < STAGES - 1; ++t)
        if (t < ntiles) issue(t);


    // Q rows of this wave as the B operand of S^T = K Q^T: lane holds Q[s0 + l32][16kk + 8g + i].
    // A negative scale is applied as |scale| on sign-flipped Q (exact), so the row max can be
    // taken on raw scores.
    s16x8 qop[KD];
    const int qi = s0 + l32;
    const float c = fabsf(a.qk_scale);
    {
        const uint16_t* qp = a.q + (int64_t)b * a.qbs + (qs.tok0 + qi) * a.qts + (int64_t)h * a.qhs;
        const short flip = a.qk_scale < 0.f ? (short)0x8000 : (short)0;
#pragma unroll
        for (int kk = 0; kk < KD; ++kk) {
            s16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
            if (qi < q_len) v = ld16(qp + 16 * kk + 8 * g);
            qop[kk] = v ^ flip;
        }
    }
    // Q and the prefetched tiles land together (one memory round trip for the prologue). No
    // load may stay outstanding into the loop: the compiler cannot count the ring's loads and
    // would drain the counter inside the loop.
    wait_vmcnt<0>();


    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    float m_i = kNegFloor, l_i = 0.f;

    for (int t = 0; t < ntiles; ++t) {
        const int n0 = wg_lo + t * BN;
        const int after = ntiles - 1 - t < STAGES - 2 ? ntiles - 1 - t : STAGES - 2;
        ring_wait<Ring::LOADS, STAGES>(after);
        barrier_lds();  // tile t landed for every wave; tile t - 1's stage is free again
        if (t + STAGES - 1 < ntiles) issue(t + STAGES - 1);
        const bool active = bs > 0 && n0 < wr.hi && n0 + BN > wr.lo;
        if (!active) continue;
        const bool masked = !(n0 >= wr.mid_lo && n0 + BN <= wr.mid_hi);
        const uint16_t* Ks = smem[t % STAGES][0];
        const uint16_t* Vs = smem[t % STAGES][1];
        // S^T = K Q^T (raw scores), 32 keys per block. Every K operand read is issued before the
        // products (left to itself the compiler reuses one register quad: read, wait, product,
        // read again, exposing the LDS latency once per product), and the two blocks'
        // accumulation chains alternate.
        f32x16 st[NB];
        s16x8 kop[NB][KD];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int row = nb * 32 + perm32(l32);
#pragma unroll
            for (int kk = 0; kk < KD; ++kk)
                kop[nb][kk] = *reinterpret_cast<const s16x8*>(Ks + row * D + (((2 * kk + g) ^ lds_swz<D>(row)) << 3));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) st[nb][r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < KD; ++kk)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) st[nb] = T::mfma32(kop[nb][kk], qop[kk], st[nb]);
        // V^T operands of O^T += V^T P^T through the LDS transpose read, issued now so that
        // they land while the softmax runs.
        const int G = lane >> 4, jj = lane & 15;
        s16x8 vop[DB][KB];
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            int col = 32 * db + 16 * (G & 1) + 4 * (jj & 3);
            const bool dvalid = col < D;
            if (!dvalid) col = col % D;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const int row = 16 * kb + 8 * (G >> 1) + (jj >> 2);
                s16x4 lo4 = ds_read_tr(Vs + lds_off<D>(row, col));
                s16x4 hi4 = ds_read_tr(Vs + lds_off<D>(row + 4, col));
                vop[db][kb] = cat4(lo4, hi4);
                if (!dvalid) vop[db][kb] = s16x8{0, 0, 0, 0, 0, 0, 0, 0};
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // Band mask, only on tiles that cross the band edge (flash_attn.py:140-145).
        // Key j is visible from this lane's query iff lo_off <= j - qi <= hi_off and j < k_len:
        // one range (register r of block nb holds key n0 + 32 nb + out_row32(r, g)); masked
        // scores become -inf.
        if (masked) {
            const int vis_lo = qi + lo_off, vis_hi = min(qi + hi_off, k_len - 1);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                float sv[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) sv[r] = st[nb][r];
                mask_runs16(sv, n0 + nb * 32 + 8 * g, vis_lo, vis_hi, 0xff800000u);
#pragma unroll
                for (int r = 0; r < 16; ++r) st[nb][r] = sv[r];
            }
        }
        // Online softmax (flash_attn.py:90-96). The row max is taken on the raw scores (c > 0)
        // and the scale is folded into one FMA per score: p = exp2(s c - m).
        // One chain per key block, each step a three-input max (v_max3): 8 NB + NB - 1
        // instructions for the 16 NB scores instead of 12 NB pairwise ones.
        float mxb[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            mxb[nb] = fmaxf(st[nb][0], st[nb][1]);
#pragma unroll
            for (int r = 2; r < 16; r += 2) mxb[nb] = fmaxf(fmaxf(mxb[nb], st[nb][r]), st[nb][r + 1]);
        }
        float mx = mxb[0];
#pragma unroll
        for (int nb = 1; nb < NB; ++nb) mx = fmaxf(mx, mxb[nb]);
        mx = max_halves(mx) * c;
        // Lazy rescaling: the running max m moves only when a tile exceeds it by more than
        // kRescaleSlack, so P stays <= 2^kRescaleSlack; O / l and the LSE use the same m, so the
        // result is unchanged while most tiles skip the O rescale entirely.
        if (__builtin_amdgcn_ballot_w64(mx > m_i + kRescaleSlack) != 0) {
            const float m_new = mx > m_i + kRescaleSlack ? mx : m_i;
            const float alpha = fast_exp2(m_i - m_new);
            l_i *= alpha;
            m_i = m_new;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
        }
        const float neg_m = -m_i;
        s16x8 pop[KB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p0 = fast_exp2(fmaf(st[nb][8 * half + 2 * i], c, neg_m));
                    const float p1 = fast_exp2(fmaf(st[nb][8 * half + 2 * i + 1], c, neg_m));
                    w[i] = T::pack2(p0, p1);
                    l_i += p0 + p1;  // fp32 row sum (flash_attn.py:96): the LSE needs it unrounded
                }
                u32x4 wv = {w[0], w[1], w[2], w[3]};
                pop[nb * 2 + half] = __builtin_bit_cast(s16x8, wv);
            }
        // O^T += V^T P^T.
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int db = 0; db < DB; ++db) acc[db] = T::mfma32(vop[db][kb], pop[kb], acc[db]);
    }

    if (bs <= 0) return;
    // Epilogue (flash_attn.py:147-154): rows that saw no key output 0 and lse = +inf.
    const float l_tot = sum_halves(l_i);
    const bool empty = l_tot == 0.f;
    const float inv = empty ? 0.f : 1.f / l_tot;
    if (qi < q_len) {
        uint16_t* op = a.o + (int64_t)b * a.obs + (qs.tok0 + qi) * a.ots + (int64_t)h * a.ohs;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const int d0 = 32 * db + 8 * rq + 4 * g;
                if (d0 < D) {
                    u32x2 w = {T::pack2(acc[db][4 * rq] * inv, acc[db][4 * rq + 1] * inv),
                               T::pack2(acc[db][4 * rq + 2] * inv, acc[db][4 * rq + 3] * inv)};
                    *reinterpret_cast<u32x2*>(op + d0) = w;
                }
            }
        if (g == 0) a.lse[(int64_t)h * a.lse_hs + qs.row0 + qi] = empty ? INFINITY : m_i + fast_log2(l_tot);
    }
}

int gcd_int(int x, int y) {
    while (y) {
        int t = x % y;
        x = y;
        y = t;
    }
    return x;
}

template <int D, int BN, int NW, int STAGES, typename T>
hipError_t launch_typed(FwdArgs args, int batch, int num_heads, int max_q, hipStream_t s) {
    args.hpw = gcd_int(args.group, NW);
    const int tpw = NW / args.hpw;
    args.gx = (max_q + tpw * 32 - 1) / (tpw * 32);
    args.gy = batch;
    args.gz = num_heads / args.hpw;
    const long long n = block_grid_size(args.gx, args.gz, args.gy, args.cu_q != nullptr);
    if (n == 0) return hipSuccess;
    if (n > (1LL << 30)) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((fwd_kernel<D, BN, NW, STAGES, T>), dim3(xcd_grid((int)n)), dim3(NW * 64), 0, s, args);
    return hipGetLastError();
}

// Tile shapes per head_dim: (keys per tile, waves per workgroup, LDS ring stages). Four-wave
// workgroups, two or more per CU: the waves sharing a SIMD then belong to different
// workgroups, whose per-tile barriers do not hold them in the same phase, so one wave's MFMAs
// overlap the other's softmax (measured 15-20% faster than eight-wave workgroups at D = 64
// and 128).
template <typename T>
hipError_t launch_dtype(const FwdArgs& args, int D, int batch, int num_heads, int max_q, hipStream_t s) {
    switch (D) {
        case 16: return launch_typed<16, 64, 4, 4, T>(args, batch, num_heads, max_q, s);
        case 32: return launch_typed<32, 64, 4, 4, T>(args, batch, num_heads, max_q, s);
        case 64: return launch_typed<64, 64, 4, 4, T>(args, batch, num_heads, max_q, s);
        case 128: return launch_typed<128, 64, 4, 2, T>(args, batch, num_heads, max_q, s);
        case 256: return launch_typed<256, 32, 4, 3, T>(args, batch, num_heads, max_q, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_fwd(const mykfa_fwd_params& p, hipStream_t stream) {
    FwdArgs a;
    a.q = static_cast<const uint16_t*>(p.q);
    a.k = static_cast<const uint16_t*>(p.k);
    a.v = static_cast<const uint16_t*>(p.v);
    a.o = static_cast<uint16_t*>(p.o);
    a.lse = p.lse;
    a.qbs = p.q_batch_stride; a.qts = p.q_token_stride; a.qhs = p.q_head_stride;
    a.kbs = p.k_batch_stride; a.kts = p.k_token_stride; a.khs = p.k_head_stride;
    a.vbs = p.v_batch_stride; a.vts = p.v_token_stride; a.vhs = p.v_head_stride;
    a.obs = p.o_batch_stride; a.ots = p.o_token_stride; a.ohs = p.o_head_stride;
    a.lse_hs = p.lse_head_stride;
    a.cu_q = p.cu_seqlens_q;
    a.cu_k = p.cu_seqlens_k;
    a.seqused_k = p.seqused_k;
    a.seqlen_q = p.max_seqlen_q;
    a.seqlen_k = p.max_seqlen_k;
    a.wl = p.window_left;
    a.wr = p.window_right;
    a.qk_scale = p.softmax_scale * 1.4426950408889634f;
    a.group = p.num_heads / p.num_kv_heads;
    a.hpw = 1;  // set per tile shape in launch_typed
    if (p.dtype == MYKFA_BF16) return launch_dtype<BF16>(a, p.head_dim, p.batch, p.num_heads, p.max_seqlen_q, stream);
    return launch_dtype<FP16>(a, p.head_dim, p.batch, p.num_heads, p.max_seqlen_q, stream);
}

}  // namespace mykfa
