// prefix_attn.hip -- MFMA flash attention of tree-verify queries over a prefix
// KV cache (the dense half of src/ragged_attn.py:1761-1798), merged into the
// ancestor walk's softmax state.
//
// Work unit: (sequence, kv head, query tile of 128 rows, prefix split).  The
// rows of a tile are (token, q head) pairs of ONE kv head's GQA group, so a
// K/V block staged in LDS (by LDS-DMA, global_load_lds_dwordx4) serves every
// q head that reads it (no repeat_kv).  Each of the 4 waves owns 32 rows as
// the N dimension of v_mfma_f32_32x32x16_{f16,bf16} products and computes,
// per 64-key block,
//   S^T = K Q^T      2 key tiles x D/16 k-steps   (16 products at D = 128)
//   O^T += V^T P^T   4 16-key steps x D/32 d-tiles (16 products at D = 128)
// Computing S transposed puts one query per lane column (lanes l and l + 32
// split its keys), so the softmax statistics need one xor-32 exchange, and
// the S^T output registers are directly the P^T operand of the next product
// (keys are permuted the same way in P^T and in the V^T operand reads).
//
// Two ways to finish:
//  * several prefix splits: each split writes its state (m, l, acc / l) to a
//    caller workspace and the tree kernels (tree_attn.hip) merge the splits,
//    walk the ancestors and normalise;
//  * one split (enough query tiles to fill the GPU): the epilogue hands the
//    state to the ancestor walk in the same workgroup, which normalises and
//    stores O -- no partial state leaves the chip.
// Split calls with fewer units than CUs use prefix_half_kernel instead
// (64-row tiles of 16-row v_mfma_f32_16x16x32 column blocks, twice the units).
#include <algorithm>
#include <mutex>

#include "qattn_common.h"
#include "qattn_device.h"
#include "tree_walk.h"

namespace qattn {

constexpr int kPrefixThreads = 256;
constexpr int kBN = 64;   // prefix keys per block
constexpr int kQB = 2;    // 16-row column blocks per wave
constexpr int kBM = 4 * 16 * kQB;  // query rows per workgroup

struct PrefixParams {
    const void* q;
    const void* kp;
    const void* vp;
    const int32_t* cu;
    float* part_m;
    float* part_l;
    void* part_acc;  // numerator / l: fp16 for fp16 inputs, else fp32 (kPartHalf)
    int64_t sq_t, sq_h;
    int64_t skp_b, skp_t, skp_h, svp_b, svp_t, svp_h;
    int64_t total_tokens;
    int32_t B, Hq, Hkv, group, max_seqlen, L;
    int32_t n_split, blocks_per_split, qtiles, n_units;
    Divider gdiv;
    Divider qtdiv, nsdiv, hkvdiv;  // qtiles, n_split, Hkv: the unit decode
    float scale_log2;
    int64_t sq_b;  // uniform batch only: per-sequence q offset (as TreeParams::sq_b)
};

// 16-byte chunk swizzle of the K/V blocks in LDS: chunk c of key row r sits at
// position c ^ kv_swz(r) of its (unpadded) row.  With 256-byte rows both
// operand reads are bank-conflict free on gfx950 (probed with
// SQ_LDS_BANK_CONFLICT): the K reads (ds_read_b128, rows 16 mt + l16, chunk
// 4 c + lq) and the V^T reads (ds_read_b64_tr_b16, 8 rows of 32 bytes per
// 32-lane pass).  Smaller head dims keep the low bits (correct, not probed).
__device__ __forceinline__ int kv_swz(int r, int dv) {
    const int b2 = (r >> 2) & 1, b3 = (r >> 3) & 1;
    return ((2 * (r & 3)) | (8 * (b3 ^ b2)) | b2) & (dv - 1);
}

// Chunk swizzle of the K/V blocks of the 32x32x16 prefix kernel: chunk c of
// key row r sits at c ^ kv_swz32(r).  Its K operand reads (ds_read_b128, 16
// consecutive rows at one chunk per 16-lane pass) need 16 distinct positions
// for rows r..r+15, which a bijection on r & 15 gives; its V^T operand reads
// (ds_read_b64_tr_b16, per 32-lane pass 4 consecutive rows x one aligned
// group of 4 chunks) need the 4 rows in distinct groups, which 4 (r & 3)
// gives.  (Positions checked on the CPU for every pass at D = 128.)
__device__ __forceinline__ int kv_swz32(int r, int dv) { return ((4 * (r & 3)) | ((r >> 2) & 3)) & (dv - 1); }

// s_waitcnt immediate (gfx9 encoding): vmcnt N, expcnt and lgkmcnt unconstrained
constexpr int kWaitVm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// One 1 KB global -> LDS load: global_load_lds_dwordx4 with a wave-uniform
// base in SGPRs and a 32-bit per-lane byte offset (lane i writes bytes
// [16 i, 16 i + 16) of the LDS run at dst), so issuing it costs no vector ALU
// work.  Written as an asm statement, which also keeps the compiler's wait
// analysis precise: it treats a pending LDS-DMA load as an out-of-order LDS
// event and would otherwise wait for every LDS read in flight
// (lgkmcnt(0)) before each use of one.  The kernel orders these loads itself
// (s_waitcnt vmcnt + barrier before a buffer is read, barrier before it is
// overwritten).
// RFL: take the base and destination through readfirstlane, for code where
// the compiler cannot prove them wave-uniform on its own (each 32-bit half
// widened as unsigned: readfirstlane returns int).
template <bool RFL = false>
__device__ __forceinline__ void lds_dma16(uint32_t voff, const char* sbase, void* dst) {
    uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)dst;
    if constexpr (RFL) {
        const uint64_t a = (uint64_t)(uintptr_t)sbase;
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
        sbase = (const char*)(uintptr_t)(((uint64_t)hi << 32) | (uint64_t)lo);
        lds = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds);
    }
    // M0 (the LDS destination) is an operand the compiler allocates ("{m0}"),
    // so it writes M0 itself and knows its value afterwards
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}

// The prefix kernel: 128-row query tiles, each wave owning 32 rows as the N
// dimension of v_mfma_f32_32x32x16 products.  Per 64-key block a wave runs
//   S^T = K Q^T      2 key tiles x D/16 k-steps   (A: K rows from LDS, B: Q in registers)
//   O^T += V^T P^T   4 16-key steps x D/32 d-tiles (A: V^T from LDS, B: P^T in registers)
// Lane l holds query l % 32; lanes l and l + 32 split the query's keys (S^T)
// and head dims (O^T), so the softmax statistics need one xor-32 exchange.
// The S^T output registers are the P^T operand: PV step (t, h) takes
// elements 8h .. 8h+7 of S tile t, i.e. keys 32t + 16h + {0..3, 8..11} on
// lanes 0-31 and + {4..7, 12..15} on lanes 32-63, and the V^T operand is
// read in that key order.
// WALK: the tree walk of the fused epilogue (heap or explicit parents, or
// none for the prefix-only pass); the split kernels leave the walk to the tree
// kernels.  DBG: the walk-export instantiation (qattn_debug_walk), which also
// writes each query's attended ancestors to tp.dbg_walk.
template <typename T, int D, bool FUSED, bool LSE, int WALK, bool BATCH, bool DBG = false>
__global__ __launch_bounds__(kPrefixThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefix_attn_kernel(
    PrefixParams p, TreeParams tp) {
    constexpr int kQB = 2;          // 16-row column blocks per wave (the epilogue's walk layout)
    constexpr int kBM = 128;        // query rows per workgroup
    constexpr int KS = D / 16;      // k-steps of S^T over the head dim
    constexpr int DT = D / 32;      // 32-row d-tiles of O^T
    constexpr int DV = D / 8;       // 16-byte chunks per key row
    constexpr int BLK = kBN * D;    // elements of one K or V block
    constexpr int NI = D / 32;      // 1 KB LDS loads per thread per K (or V) block
    constexpr int RPI = 512 / D;    // key rows per 1 KB load
    static_assert(NI * 4 * 512 == BLK, "a block is 4 waves x NI loads of 1 KB");
    // Double buffers of the K and V blocks, four LDS variables so that the
    // compiler tells them apart: a read of one buffer does not wait for the
    // LDS-DMA loads in flight into another.
    __shared__ __attribute__((aligned(1024))) uint16_t Kb0[BLK], Kb1[BLK], Vb0[BLK], Vb1[BLK];
    // DBG only: the node of each row the epilogue stages in LDS
    __shared__ int32_t dbg_slot[DBG ? 2 * (BLK / D) : 1];
    auto kbuf = [&](auto i) -> uint16_t* {
        if constexpr (decltype(i)::value == 0) return Kb0; else return Kb1;
    };
    auto vbuf = [&](auto i) -> uint16_t* {
        if constexpr (decltype(i)::value == 0) return Vb0; else return Vb1;
    };

    // Logical unit order puts the query tiles of one (sequence, kv head, split)
    // next to each other; hardware deals blockIdx round-robin over the 8 XCDs,
    // so unit u runs on XCD (blockIdx % 8) and a K/V block is shared in one L2.
    const int per = gridDim.x >> 3;
    const int unit = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (unit >= p.n_units) return;
    // (magic-number divisions: the generic 32-bit ones held the first loads
    // of a short launch back)
    const int r0 = divide(unit, p.qtdiv);
    const int qt = unit - r0 * p.qtiles;
    const int r1 = divide(r0, p.nsdiv);
    const int split = r0 - r1 * p.n_split;
    const int seq = divide(r1, p.hkvdiv);
    const int kvh = r1 - seq * p.Hkv;

    // (BATCH: a uniform batch of max_seqlen rows per sequence, no cu)
    const int32_t s0 = BATCH ? seq * p.max_seqlen : p.cu[seq];
    const int32_t s1 = BATCH ? s0 + p.max_seqlen : p.cu[seq + 1];
    if (s0 < 0 || s1 < s0 || (int64_t)s1 > p.total_tokens) return;
    int32_t n = s1 - s0;
    if (n > p.max_seqlen) n = p.max_seqlen;
    const int g = p.group;
    const int rows = n * g;
    if (qt * kBM >= rows) return;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int q32 = lane & 31, hl = lane >> 5;

    // this lane's query row (B operand column, output column), recomputed
    // after the key loop rather than kept live through it
    auto query_of = [&](int64_t& qrow, int& qh) {
        const int rr = qt * kBM + wave * 32 + q32;
        const int tok = divide(rr, p.gdiv);
        qh = kvh * g + (rr - tok * g);
        qrow = (int64_t)s0 + tok;
        return rr < rows;
    };
    // Q^T operand of step s: dims 16 s + 8 hl .. + 7 of the lane's query
    Vec16 qf[KS];
    {
        int64_t qrow;
        int qh;
        const bool valid = query_of(qrow, qh);
        const uint16_t* qp = (const uint16_t*)p.q + qrow * p.sq_t + (BATCH ? (int64_t)seq * p.sq_b : 0) +
                             (int64_t)qh * p.sq_h + 8 * hl;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            qf[s] = Vec16{{0u, 0u, 0u, 0u}};
            if (valid) qf[s] = ld16(qp + 16 * s);
        }
    }

    const int k_lo = split * p.blocks_per_split * kBN;
    const int k_hi = (k_lo + p.blocks_per_split * kBN < p.L) ? k_lo + p.blocks_per_split * kBN : p.L;
    const int nb = (k_hi - k_lo + kBN - 1) / kBN;  // >= 1: every split holds a key
    const char* kbase = (const char*)((const uint16_t*)p.kp + (int64_t)seq * p.skp_b + (int64_t)kvh * p.skp_h);
    const char* vbase = (const char*)((const uint16_t*)p.vp + (int64_t)seq * p.svp_b + (int64_t)kvh * p.svp_h);
    const int64_t kst = 2 * p.skp_t, vst = 2 * p.svp_t;  // bytes between keys

    float m_run = -INFINITY, l_run = 0.f;  // l_run: this lane's half of the keys
    f16v_t oacc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;

    // ---- K/V blocks go straight from global memory to LDS (global_load_lds,
    // 16 bytes per lane, lane i of a load writes bytes [16 i, 16 i + 16) of its
    // 1 KB): load i of wave w covers key rows (w NI + i) RPI .. + RPI - 1, and
    // each lane fetches the chunk that the swizzle puts at its position ----
    // Byte offsets of this lane's loads within a block: 32-bit (the host checks
    // that 64 key rows span less than 4 GB), added to the block's uniform base.
    uint32_t koff[NI], voff[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = (wave * NI + i) * RPI + lane / DV;
        const uint32_t col = 16 * ((lane % DV) ^ kv_swz32(row, DV));
        koff[i] = (uint32_t)row * (uint32_t)kst + col;
        voff[i] = (uint32_t)row * (uint32_t)vst + col;
    }
    auto issue = [&](const char* base, int64_t st, const uint32_t (&off)[NI], int j, uint16_t* buf) {
        const int kb = k_lo + j * kBN;
        const char* gb = base + (int64_t)kb * st;
        if (__builtin_expect(kb + kBN <= k_hi, 1)) {
#pragma unroll
            for (int i = 0; i < NI; ++i) lds_dma16(off[i], gb, buf + (wave * NI + i) * 512);
        } else {
            // tail block of the split: rows past k_hi - 1 load that key instead
            const int last = k_hi - 1 - kb;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int row = (wave * NI + i) * RPI + lane / DV;
                const uint32_t col = 16 * ((lane % DV) ^ kv_swz32(row, DV));
                lds_dma16((uint32_t)min(row, last) * (uint32_t)st + col, gb, buf + (wave * NI + i) * 512);
            }
        }
    };
    auto issue_k = [&](int j, auto buf) { issue(kbase, kst, koff, j, kbuf(buf)); };
    auto issue_v = [&](int j, auto buf) { issue(vbase, vst, voff, j, vbuf(buf)); };

    // Operand read addresses (elements).  K (A of S^T, step s, key tile t):
    // row 32 t + q32, chunk 2 s + hl: (kaddr0 ^ 16 s) + 32 D t (the swizzle
    // flips only chunk bits, which the row base leaves clear).  V^T (A of
    // O^T, 16-key step th = 2t + h, d-tile dt): two ds_read_b64_tr_b16, X for
    // keys 16 th + 4 hl + 0..3 and Y for + 8; within each 16-lane group lane
    // j points at row key0 + j / 4, dims 32 dt + 16 ((lane >> 4) & 1) +
    // 4 (j % 4) .. + 3, and receives keys key0 + 0..3 at dim 32 dt + q32.
    const int kaddr0 = q32 * D + 8 * (hl ^ kv_swz32(q32, DV));
    int vx0, vy0;
    {
        const int rx = 4 * hl + ((lane & 15) >> 2), ry = rx + 8;
        const int cx = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
        vx0 = rx * D + 8 * (cx ^ kv_swz32(rx, DV)) + 4 * (lane & 1);
        vy0 = ry * D + 8 * (cx ^ kv_swz32(ry, DV)) + 4 * (lane & 1);
    }

    // S^T = K Q^T of the block in K buffer buf; step i = (k-step i / 2, key
    // tile i % 2), so consecutive products write different tiles, and the K
    // operand of step i + 1 is read before the product of step i is issued.
    auto s_product = [&](auto buf, f16v_t (&s)[2]) {
        const uint16_t* kb = kbuf(buf);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
        constexpr int NS = 2 * KS;
        auto fetch = [&](int i) { return ld16(kb + (kaddr0 ^ (16 * (i >> 1))) + 32 * D * (i & 1)); };
        Vec16 ka[3];
        ka[0] = fetch(0);
        ka[1] = fetch(1);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if (i + 2 < NS) ka[(i + 2) % 3] = fetch(i + 2);
            s[i & 1] = mma32<T>(ka[i % 3], qf[i >> 1], s[i & 1]);
        }
    };

    // Online softmax of one block (the lane's query; keys 32 t + 8 (r / 4) +
    // 4 hl + r % 4 of element r of tile t).  The running max is kept on raw
    // scores q.k (scale > 0 keeps the order) and scale*log2(e) is folded into
    // the exponent: p = exp2(s c - m c), one FMA.  Lazy rescaling: the
    // exponent reference m_run only moves when a block max exceeds it by more
    // than kLazy/c (a factor 2^kLazy in P), so the accumulators are rescaled on
    // a handful of blocks.  P stays <= 2^kLazy and l carries the same
    // reference.  The PV product rounds P to the input type while l sums it
    // unrounded, so the largest weight is exact only when it is 1: bf16 (8
    // mantissa bits) therefore moves the reference on every new maximum, as
    // the reference's FA2 loop does; fp16 (11 bits) keeps the lazy reference.
    const float csc = p.scale_log2;
    auto softmax = [&](f16v_t (&s)[2], Vec16 (&pf)[4], float& alpha, bool& rescale, int kb, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        constexpr float kLazy = T::kCode == QATTN_DTYPE_BF16 ? 0.f : 8.f;
        if constexpr (MASK) {  // tail block of the split: keys at or beyond k_hi do not exist
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (kb + 32 * t + 8 * (r >> 2) + 4 * hl + (r & 3) >= k_hi) s[t][r] = -INFINITY;
        }
        float mb = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) mb = fmaxf(mb, s[t][r]);
        mb = xor32_max(mb);
        const bool move = (mb - m_run) * csc > kLazy;  // always true on the first block
        const float m_new = move ? mb : m_run;
        alpha = move ? fast_exp2((m_run - m_new) * csc) : 1.f;  // m_run = -inf: 0
        rescale |= move;
        const float mc = m_new * csc;
        float psum = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float e = fast_exp2(__builtin_fmaf(s[t][r], csc, -mc));
                s[t][r] = e;
                psum += e;
            }
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    pf[2 * t + h].w[i] = MfmaOps<T>::pack2(s[t][8 * h + 2 * i], s[t][8 * h + 2 * i + 1]);
    };
    auto rescale_o = [&](float alpha, bool rescale) {
        // the accumulators need rescaling only when some running max moved
        if (__builtin_expect(__any(rescale), 0)) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
        }
    };

    // O^T += V^T P^T of the block in V buffer buf; step i = (16-key step
    // i / DT, d-tile i % DT), operands read one step ahead
    auto pv_product = [&](auto buf, const Vec16 (&pf)[4]) {
        typedef short v4s __attribute__((ext_vector_type(4)));
        const uint16_t* vb = vbuf(buf);
        auto fetch = [&](int i) {
            const int th = i / DT, dt = i % DT;
            const uint16_t* ax = vb + (vx0 ^ (32 * dt)) + 16 * D * th;
            const uint16_t* ay = vb + (vy0 ^ (32 * dt)) + 16 * D * th;
            const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)ax);
            const v4s y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)ay);
            const uint2 x2 = __builtin_bit_cast(uint2, x), y2 = __builtin_bit_cast(uint2, y);
            return Vec16{{x2.x, x2.y, y2.x, y2.y}};
        };
        constexpr int NS = 4 * DT;
        Vec16 va[3];
        va[0] = fetch(0);
        if (NS > 1) va[1] = fetch(1);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if (i + 2 < NS) va[(i + 2) % 3] = fetch(i + 2);
            oacc[i % DT] = mma32<T>(va[i % 3], pf[i / DT], oacc[i % DT]);
        }
    };

    // ---- pipeline over the split's blocks j = 0 .. nb-1: iteration j starts
    // after a barrier that publishes K_{j+1} and V_j, issues V_{j+1} and
    // K_{j+2} into the buffers freed by the barrier, forms S_{j+1} on the
    // matrix cores while the softmax of block j runs on the vector ALUs, and
    // ends with the PV product of block j ----
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    issue_k(0, B0{});
    issue_v(0, B0{});
    if (nb > 1) {
        issue_k(1, B1{});
        __builtin_amdgcn_s_waitcnt(kWaitVm(NI));  // K_0 and V_0 (and Q) have landed
    } else {
        __builtin_amdgcn_s_waitcnt(kWaitVm(0));
    }
    __syncthreads();
    f16v_t sc[2];
    s_product(B0{}, sc);
    // block j uses K buffer j & 1 and V buffer j & 1; the loop is unrolled by
    // two so every buffer choice is a compile-time constant
    auto step = [&](int j, auto par) {
        constexpr int P = decltype(par)::value;
        using Pn = std::integral_constant<int, P ^ 1>;
        __builtin_amdgcn_s_waitcnt(kWaitVm(0));
        __syncthreads();
        issue_v(j + 1, Pn{});
        if (j + 2 < nb) issue_k(j + 2, par);
        f16v_t sn[2];
        Vec16 pf[4];
        float alpha;
        bool rescale = false;
        softmax(sc, pf, alpha, rescale, k_lo + j * kBN, std::false_type{});
        s_product(Pn{}, sn);
        rescale_o(alpha, rescale);
        pv_product(par, pf);
        sc[0] = sn[0];
        sc[1] = sn[1];
    };
    for (int j = 0; j + 1 < nb; j += 2) {
        step(j, B0{});
        if (j + 2 < nb) step(j + 1, B1{});
    }
    {
        __builtin_amdgcn_s_waitcnt(kWaitVm(0));
        __syncthreads();
        const int kb = k_lo + (nb - 1) * kBN;
        Vec16 pf[4];
        float alpha;
        bool rescale = false;
        if (kb + kBN > k_hi)
            softmax(sc, pf, alpha, rescale, kb, std::true_type{});
        else
            softmax(sc, pf, alpha, rescale, kb, std::false_type{});
        rescale_o(alpha, rescale);
        if ((nb - 1) & 1)
            pv_product(B1{}, pf);
        else
            pv_product(B0{}, pf);
    }
    __syncthreads();  // the LDS is reused by the fused epilogue

    const float l_tot = xor32_sum(l_run);  // both halves of the query's keys
    m_run *= p.scale_log2;                 // to the log2 units of the tree walk's scores

    if constexpr (!FUSED) {
        // ---- partial state of this split: (m, l, acc / l).  For fp16
        // inputs the normalised numerator is stored in fp16, which halves the
        // bytes the merge reads, as the reference's own split pipelines hand
        // fp16 partial outputs to their merge (scripts/benchmark_micro.py:
        // 576-592, src/ragged_attn.py:1619); bf16 inputs keep fp32 states.
        // Element 4 j + e of d-tile dt is dim 32 dt + 8 j + 4 hl + e. ----
        int64_t qrow;
        int qh;
        if (query_of(qrow, qh)) {
            const int64_t plane = p.total_tokens * (int64_t)p.Hq;
            const int64_t idx = (int64_t)split * plane + qrow * p.Hq + qh;
            if (hl == 0) {
                p.part_m[idx] = m_run;
                p.part_l[idx] = l_tot;
            }
            const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
            const int64_t off = idx * D + 4 * hl;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const float a = oacc[dt][4 * jj] * inv, b = oacc[dt][4 * jj + 1] * inv;
                    const float c = oacc[dt][4 * jj + 2] * inv, d = oacc[dt][4 * jj + 3] * inv;
                    if constexpr (kPartHalf<T>)
                        *reinterpret_cast<uint2*>((uint16_t*)p.part_acc + off + 32 * dt + 8 * jj) =
                            make_uint2(MfmaOps<F16>::pack2(a, b), MfmaOps<F16>::pack2(c, d));
                    else
                        *reinterpret_cast<float4*>((float*)p.part_acc + off + 32 * dt + 8 * jj) = make_float4(a, b, c, d);
                }
            }
        }
    } else {
        // ---- fused epilogue: each wave re-lays its 32 rows in its own LDS
        // buffer as 4 lanes per query (no other wave reads it, so only the
        // wave's own LDS order matters), takes m and l by shuffles, and runs
        // the ancestor walks of its two 16-row blocks with their loads
        // interleaved ----
        constexpr int NCH = D / 32;
        constexpr int C4 = D / 4;  // float4 per staged row; float4 c of row r sits at c ^ (r & 7)
        uint16_t* wbuf = wave == 0 ? Kb0 : (wave == 1 ? Kb1 : (wave == 2 ? Vb0 : Vb1));
        float4* Os = reinterpret_cast<float4*>(wbuf);  // [32 rows][C4]
        static_assert(32 * D * 4 <= BLK * 2, "epilogue staging must fit one K/V buffer");
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                Os[q32 * C4 + ((8 * dt + 2 * jj + hl) ^ (q32 & 7))] = make_float4(
                    oacc[dt][4 * jj], oacc[dt][4 * jj + 1], oacc[dt][4 * jj + 2], oacc[dt][4 * jj + 3]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int grp = lane >> 2, j = lane & 3;
        float acc[kQB][8 * NCH], mw[kQB], lw[kQB];
        int tokb[kQB], hb[kQB];
        int64_t qrb[kQB];
        bool vb[kQB];
        Vec16 qf4[kQB][NCH];
#pragma unroll
        for (int b = 0; b < kQB; ++b) {
            const int rr = qt * kBM + wave * (16 * kQB) + 16 * b + grp;
            vb[b] = rr < rows;
            // a row past the tile's queries walks the tile's first token (valid
            // memory, ancestors inside the staged ranges) and stores nothing
            tokb[b] = vb[b] ? divide(rr, p.gdiv) : (qt * kBM) / g;
            hb[b] = kvh * g + (vb[b] ? rr - tokb[b] * g : 0);
            qrb[b] = (int64_t)s0 + tokb[b];
            const int row = 16 * b + grp;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const float4 a0 = Os[row * C4 + ((2 * (j + 4 * i)) ^ (row & 7))];
                const float4 a1 = Os[row * C4 + ((2 * (j + 4 * i) + 1) ^ (row & 7))];
                acc[b][8 * i + 0] = a0.x;
                acc[b][8 * i + 1] = a0.y;
                acc[b][8 * i + 2] = a0.z;
                acc[b][8 * i + 3] = a0.w;
                acc[b][8 * i + 4] = a1.x;
                acc[b][8 * i + 5] = a1.y;
                acc[b][8 * i + 6] = a1.z;
                acc[b][8 * i + 7] = a1.w;
            }
            // query 16 b + grp's state is held by lane 16 b + grp of the MFMA layout
            mw[b] = __shfl(m_run, 16 * b + grp);
            lw[b] = __shfl(l_tot, 16 * b + grp);
            if constexpr (WALK != WALK_NONE) load_q4<D, BATCH>(tp, seq, qrb[b], hb[b], j, qf4[b]);
        }
        if constexpr (WALK != WALK_NONE) {  // (prefix only: nothing to walk)
        // Heap parents are monotonic, so walk step t of every token in the
        // tile's range [tl, th] lies in [par^t(tl), par^t(th)].  When those
        // ranges (steps 1 ..) total at most 128 rows they are staged once in
        // LDS, level after level (K rows in Kb0/Kb1, V rows in Vb0/Vb1, 64 rows
        // per buffer), and the walks read them there; each query's own row
        // (step 0) comes from global memory.  Otherwise the walks gather every
        // step from global memory.
        // (The explicit-parents walk has no such ranges and always gathers.)
        constexpr int kRowsPerBuf = BLK / D;
        constexpr int kLdsRows = 2 * kRowsPerBuf;
        const int tl = (qt * kBM) / g;
        const int th = (min(qt * kBM + kBM, rows) - 1) / g;
        int nlev = 0, total = WALK == WALK_HEAP ? 0 : kLdsRows + 1;
        if constexpr (WALK == WALK_HEAP) {
            int lo = tl, hi = th;
            for (int t = 1; t <= tp.max_depth && total <= kLdsRows; ++t) {
                if (lo == 0 && hi == 0) break;  // past the root every step is a self-loop
                lo = heap_parent(lo, tp.bdiv);
                hi = heap_parent(hi, tp.bdiv);
                total += hi - lo + 1;
                nlev = t;
            }
        }
        // (DBG: lane 0 of each query's group owns the query's export row)
        int32_t* dbg[kQB] = {};
        if constexpr (DBG) {
#pragma unroll
            for (int b = 0; b < kQB; ++b) {
                if (vb[b] && j == 0) {
                    dbg[b] = tp.dbg_walk + (qrb[b] * tp.Hq + hb[b]) * (tp.max_depth + 1);
                    for (int i = 0; i <= tp.max_depth; ++i) dbg[b][i] = -1;
                }
            }
        }
        if (WALK == WALK_HEAP && total <= kLdsRows) {
            const int64_t kvb = kv_base(tp, seq, s0);
            const uint16_t* kg = (const uint16_t*)tp.k + (int64_t)kvh * tp.sk_h;
            const uint16_t* vg = (const uint16_t*)tp.v + (int64_t)kvh * tp.sv_h;
            auto krow = [&](int slot) { return (slot < kRowsPerBuf ? Kb0 : Kb1) + (slot % kRowsPerBuf) * D; };
            auto vrow = [&](int slot) { return (slot < kRowsPerBuf ? Vb0 : Vb1) + (slot % kRowsPerBuf) * D; };
            // step 0 loads go out before the staging
            Vec16 k0[kQB][NCH], v0[kQB][NCH];
#pragma unroll
            for (int b = 0; b < kQB; ++b)
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    k0[b][i] = ld16(kg + (kvb + tokb[b]) * tp.sk_t + 8 * j + 32 * i);
                    v0[b][i] = ld16(vg + (kvb + tokb[b]) * tp.sv_t + 8 * j + 32 * i);
                }
            __syncthreads();  // every wave has read its staged O
            {
                int lo = tl, hi = th, off = 0;
                for (int t = 1; t <= nlev; ++t) {
                    lo = heap_parent(lo, tp.bdiv);
                    hi = heap_parent(hi, tp.bdiv);
                    const int sz = hi - lo + 1;
                    for (int idx = tid; idx < sz * DV; idx += kPrefixThreads) {
                        const int r = idx / DV, c = idx - r * DV;
                        const int64_t grow = kvb + lo + r;
                        st16(krow(off + r) + 8 * c, ld16(kg + grow * tp.sk_t + 8 * c));
                        st16(vrow(off + r) + 8 * c, ld16(vg + grow * tp.sv_t + 8 * c));
                        if constexpr (DBG) {
                            if (c == 0) dbg_slot[off + r] = lo + r;
                        }
                    }
                    off += sz;
                }
            }
            __syncthreads();
            int32_t cur[kQB], prev[kQB];
#pragma unroll
            for (int b = 0; b < kQB; ++b) {
                float sc = qk4<T, NCH>(qf4[b], k0[b]) * tp.scale_log2;
                fold_scores<T, NCH, 1>(&sc, &v0[b], mw[b], lw[b], acc[b]);
                if constexpr (DBG) {
                    if (dbg[b]) dbg[b][0] = tokb[b];
                }
                prev[b] = tokb[b];
                cur[b] = heap_parent(tokb[b], tp.bdiv);
            }
            int lo = tl, hi = th, off = 0;
            for (int t = 1; t <= nlev; ++t) {
                lo = heap_parent(lo, tp.bdiv);
                hi = heap_parent(hi, tp.bdiv);
#pragma unroll
                for (int b = 0; b < kQB; ++b) {
                    const int slot = off + cur[b] - lo;  // inside [off, off + hi - lo] by monotonicity
                    Vec16 kk[NCH], vv[1][NCH];
#pragma unroll
                    for (int i = 0; i < NCH; ++i) {
                        kk[i] = ld16(krow(slot) + 8 * j + 32 * i);
                        vv[0][i] = ld16(vrow(slot) + 8 * j + 32 * i);
                    }
                    float sc = qk4<T, NCH>(qf4[b], kk) * tp.scale_log2;
                    sc = cur[b] != prev[b] ? sc : -INFINITY;  // the root's self-loop is not a step
                    fold_scores<T, NCH, 1>(&sc, vv, mw[b], lw[b], acc[b]);
                    if constexpr (DBG) {
                        if (dbg[b]) dbg[b][t] = cur[b] != prev[b] ? dbg_slot[slot] : -1;
                    }
                    prev[b] = cur[b];
                    cur[b] = heap_parent(cur[b], tp.bdiv);
                }
                off += hi - lo + 1;
            }
        } else {
            // steps per chunk of each walk: half the single-walk chunk from
            // D = 64 up (two full chunks in flight spill registers there)
            constexpr int CH1 = 8 / NCH;
            constexpr int CHW = D >= 64 ? CH1 / 2 : CH1;
            using W = Walk4<T, D, WALK, KV_PACKED, CHW, BATCH, DBG>;
            W w0(tp, seq, s0, n, tokb[0], kvh, j, nullptr, dbg[0]), w1(tp, seq, s0, n, tokb[1], kvh, j, nullptr, dbg[1]);
            w0.issue();
            w1.issue();
            w0.fold(qf4[0], mw[0], lw[0], acc[0]);
            w1.fold(qf4[1], mw[1], lw[1], acc[1]);
            for (;;) {
                const bool a0 = w0.more(), a1 = w1.more();
                if (!a0 && !a1) break;
                if (a0) w0.issue();
                if (a1) w1.issue();
                if (a0) w0.fold(qf4[0], mw[0], lw[0], acc[0]);
                if (a1) w1.fold(qf4[1], mw[1], lw[1], acc[1]);
            }
        }
        }
#pragma unroll
        for (int b = 0; b < kQB; ++b)
            if (vb[b]) write_out4<T, D, LSE, BATCH>(tp, seq, qrb[b], hb[b], j, mw[b], lw[b], acc[b]);
    }
}


// Half-height split kernel: 64-row query tiles, one 16-row column block per
// wave, v_mfma_f32_16x16x32 products, partial states only.  It serves split
// calls whose units would leave CUs idle (a decode step of a small tree):
// half the rows per unit gives twice the units.
template <typename T, int D, bool BATCH>
__global__ __launch_bounds__(kPrefixThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefix_half_kernel(
    PrefixParams p) {
    constexpr int QB = 1;
    constexpr int kQB = QB;         // (hides the namespace default) column blocks per wave
    constexpr int kBM = 64 * QB;    // query rows per workgroup
    constexpr int NC = D / 32;      // MFMA k-chunks over the head dim
    constexpr int ND = D / 16;      // output tiles over the head dim
    constexpr int DV = D / 8;       // 16-byte chunks per key row
    constexpr int BLK = kBN * D;    // elements of one K or V block
    constexpr int NI = D / 32;      // 1 KB LDS loads per thread per K (or V) block
    constexpr int RPI = 512 / D;    // key rows per 1 KB load
    static_assert(NI * 4 * 512 == BLK, "a block is 4 waves x NI loads of 1 KB");
    // Double buffers of the K and V blocks, four LDS variables so that the
    // compiler tells them apart: a read of one buffer does not wait for the
    // LDS-DMA loads in flight into another.
    __shared__ __attribute__((aligned(1024))) uint16_t Kb0[BLK], Kb1[BLK], Vb0[BLK], Vb1[BLK];
    auto kbuf = [&](auto i) -> uint16_t* {
        if constexpr (decltype(i)::value == 0) return Kb0; else return Kb1;
    };
    auto vbuf = [&](auto i) -> uint16_t* {
        if constexpr (decltype(i)::value == 0) return Vb0; else return Vb1;
    };

    // Logical unit order puts the query tiles of one (sequence, kv head, split)
    // next to each other; hardware deals blockIdx round-robin over the 8 XCDs,
    // so unit u runs on XCD (blockIdx % 8) and a K/V block is shared in one L2.
    const int per = gridDim.x >> 3;
    const int unit = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (unit >= p.n_units) return;
    // (magic-number divisions: the generic 32-bit ones held the first loads
    // of a short launch back)
    const int r0 = divide(unit, p.qtdiv);
    const int qt = unit - r0 * p.qtiles;
    const int r1 = divide(r0, p.nsdiv);
    const int split = r0 - r1 * p.n_split;
    const int seq = divide(r1, p.hkvdiv);
    const int kvh = r1 - seq * p.Hkv;

    // (BATCH: a uniform batch of max_seqlen rows per sequence, no cu)
    const int32_t s0 = BATCH ? seq * p.max_seqlen : p.cu[seq];
    const int32_t s1 = BATCH ? s0 + p.max_seqlen : p.cu[seq + 1];
    if (s0 < 0 || s1 < s0 || (int64_t)s1 > p.total_tokens) return;
    int32_t n = s1 - s0;
    if (n > p.max_seqlen) n = p.max_seqlen;
    const int g = p.group;
    const int rows = n * g;
    if (qt * kBM >= rows) return;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int l16 = lane & 15;
    const int lq = lane >> 4;

    // this lane's query rows (B operand column / output column), one per block
    // (token row, q head) of this lane's query in column block b (recomputed
    // after the key loop rather than kept live through it)
    auto query_of = [&](int b, int64_t& qrow, int& qh) {
        const int rr = qt * kBM + wave * (16 * kQB) + 16 * b + l16;
        const int tok = divide(rr, p.gdiv);
        qh = kvh * g + (rr - tok * g);
        qrow = (int64_t)s0 + tok;
        return rr < rows;
    };
    Vec16 qf[kQB][NC];
#pragma unroll
    for (int b = 0; b < kQB; ++b) {
        int64_t qrow;
        int qh;
        const bool valid = query_of(b, qrow, qh);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            qf[b][c] = Vec16{{0u, 0u, 0u, 0u}};
            if (valid)
                qf[b][c] = ld16((const uint16_t*)p.q + qrow * p.sq_t + (BATCH ? (int64_t)seq * p.sq_b : 0) +
                                (int64_t)qh * p.sq_h +
                                32 * c + 8 * lq);
        }
    }

    const int k_lo = split * p.blocks_per_split * kBN;
    const int k_hi = (k_lo + p.blocks_per_split * kBN < p.L) ? k_lo + p.blocks_per_split * kBN : p.L;
    const int nb = (k_hi - k_lo + kBN - 1) / kBN;  // >= 1: every split holds a key
    const char* kbase = (const char*)((const uint16_t*)p.kp + (int64_t)seq * p.skp_b + (int64_t)kvh * p.skp_h);
    const char* vbase = (const char*)((const uint16_t*)p.vp + (int64_t)seq * p.svp_b + (int64_t)kvh * p.svp_h);
    const int64_t kst = 2 * p.skp_t, vst = 2 * p.svp_t;  // bytes between keys

    float m_run[kQB], l_run[kQB];
    f4_t oacc[kQB][ND];
#pragma unroll
    for (int b = 0; b < kQB; ++b) {
        m_run[b] = -INFINITY;
        l_run[b] = 0.f;
#pragma unroll
        for (int i = 0; i < ND; ++i) oacc[b][i] = f4_t{0.f, 0.f, 0.f, 0.f};
    }

    // ---- K/V blocks go straight from global memory to LDS (global_load_lds,
    // 16 bytes per lane, lane i of a load writes bytes [16 i, 16 i + 16) of its
    // 1 KB): load i of wave w covers key rows (w NI + i) RPI .. + RPI - 1, and
    // each lane fetches the chunk that the swizzle puts at its position ----
    // Byte offsets of this lane's loads within a block: 32-bit (the host checks
    // that 64 key rows span less than 4 GB), added to the block's uniform base.
    uint32_t koff[NI], voff[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = (wave * NI + i) * RPI + lane / DV;
        const uint32_t col = 16 * ((lane % DV) ^ kv_swz(row, DV));
        koff[i] = (uint32_t)row * (uint32_t)kst + col;
        voff[i] = (uint32_t)row * (uint32_t)vst + col;
    }
    auto issue = [&](const char* base, int64_t st, const uint32_t (&off)[NI], int j, uint16_t* buf) {
        const int kb = k_lo + j * kBN;
        const char* gb = base + (int64_t)kb * st;
        if (__builtin_expect(kb + kBN <= k_hi, 1)) {
#pragma unroll
            for (int i = 0; i < NI; ++i) lds_dma16<QB == 1>(off[i], gb, buf + (wave * NI + i) * 512);
        } else {
            // tail block of the split: rows past k_hi - 1 load that key instead
            const int last = k_hi - 1 - kb;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int row = (wave * NI + i) * RPI + lane / DV;
                const uint32_t col = 16 * ((lane % DV) ^ kv_swz(row, DV));
                lds_dma16<QB == 1>((uint32_t)min(row, last) * (uint32_t)st + col, gb, buf + (wave * NI + i) * 512);
            }
        }
    };
    auto issue_k = [&](int j, auto buf) { issue(kbase, kst, koff, j, kbuf(buf)); };
    auto issue_v = [&](int j, auto buf) { issue(vbase, vst, voff, j, vbuf(buf)); };

    // operand read addresses (elements): K row 16 mt + l16, chunk 4 c + lq;
    // V^T through ds_read_b64_tr_b16: lane j of 16-lane group lq reads key row
    // 32 kc + 16 h + 4 lq + j / 4 at dims 16 dt + 4 (j % 4) .. + 3, and receives
    // keys 32 kc + 16 h + 4 lq + 0..3 at dim 16 dt + j -- the key order of the
    // P^T operand formed from the S^T output registers.  The V^T address of
    // d-tile dt is vaddr0 ^ (16 dt): the swizzle flips only chunk bits, which
    // the row base leaves clear.
    int kaddr[NC];
    int vaddr0;
    {
        const int sk = kv_swz(l16, DV);
#pragma unroll
        for (int c = 0; c < NC; ++c) kaddr[c] = l16 * D + 8 * ((4 * c + lq) ^ sk);
        const int vr = 4 * lq + (l16 >> 2);
        vaddr0 = vr * D + 8 * (((l16 & 3) >> 1) ^ kv_swz(vr, DV)) + 4 * (l16 & 1);
    }

    // S^T = K Q^T of the block in K buffer kbuf: lane holds keys 16 mt + 4 lq + i
    // of query l16.  Step i = (c, mt); the K operand of step i + 1 is read
    // before the products of step i are issued.
    auto s_product = [&](auto buf, f4_t (&s)[kQB][4]) {
        const uint16_t* kb = kbuf(buf);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int b = 0; b < kQB; ++b) s[b][mt] = f4_t{0.f, 0.f, 0.f, 0.f};
        constexpr int NS = 4 * NC;
        Vec16 ka[2];
        ka[0] = ld16(kb + kaddr[0]);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if (i + 1 < NS) {
                const int c1 = (i + 1) / 4, mt1 = (i + 1) % 4;
                ka[(i + 1) & 1] = ld16(kb + kaddr[c1] + 16 * D * mt1);
            }
            const int cc = i / 4, mt = i % 4;
#pragma unroll
            for (int b = 0; b < kQB; ++b) s[b][mt] = MfmaOps<T>::mma(ka[i & 1], qf[b][cc], s[b][mt]);
        }
    };

    // Online softmax of one block, per column block.  The running max is kept
    // on raw scores q.k (scale > 0 keeps the order) and scale*log2(e) is folded
    // into the exponent: p = exp2(s c - m c), one FMA.  Lazy rescaling: the
    // exponent reference m_run only moves when a block max exceeds it by more
    // than kLazy/c (a factor 2^kLazy in P), so the accumulators are rescaled on
    // a handful of blocks.  P stays <= 2^kLazy and l carries the same
    // reference.  The PV product rounds P to the input type while l sums it
    // unrounded, so the largest weight is exact only when it is 1: bf16 (8
    // mantissa bits) therefore moves the reference on every new maximum, as
    // the reference's FA2 loop does; fp16 (11 bits) keeps the lazy reference.
    const float csc = p.scale_log2;
    auto softmax = [&](f4_t (&s)[kQB][4], Vec16 (&pf)[kQB][2], float (&alpha)[kQB], bool& rescale, int kb,
                       auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        constexpr float kLazy = T::kCode == QATTN_DTYPE_BF16 ? 0.f : 8.f;
        if constexpr (MASK) {  // tail block of the split: keys at or beyond k_hi do not exist
#pragma unroll
            for (int b = 0; b < kQB; ++b)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (kb + 16 * mt + 4 * lq + i >= k_hi) s[b][mt][i] = -INFINITY;
        }
#pragma unroll
        for (int b = 0; b < kQB; ++b) {
            float mb = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) mb = fmaxf(mb, s[b][mt][i]);
            mb = col4_max(mb);
            const bool move = (mb - m_run[b]) * csc > kLazy;  // always true on the first block
            const float m_new = move ? mb : m_run[b];
            alpha[b] = move ? fast_exp2((m_run[b] - m_new) * csc) : 1.f;  // m_run = -inf: 0
            rescale |= move;
            const float mc = m_new * csc;
            float psum = 0.f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = fast_exp2(__builtin_fmaf(s[b][mt][i], csc, -mc));
                    s[b][mt][i] = e;
                    psum += e;
                }
            }
            l_run[b] = l_run[b] * alpha[b] + psum;
            m_run[b] = m_new;
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                pf[b][kc].w[0] = MfmaOps<T>::pack2(s[b][2 * kc][0], s[b][2 * kc][1]);
                pf[b][kc].w[1] = MfmaOps<T>::pack2(s[b][2 * kc][2], s[b][2 * kc][3]);
                pf[b][kc].w[2] = MfmaOps<T>::pack2(s[b][2 * kc + 1][0], s[b][2 * kc + 1][1]);
                pf[b][kc].w[3] = MfmaOps<T>::pack2(s[b][2 * kc + 1][2], s[b][2 * kc + 1][3]);
            }
        }
    };
    auto rescale_o = [&](const float (&alpha)[kQB], bool rescale) {
        // the accumulators need rescaling only when some running max moved
        if (__builtin_expect(__any(rescale), 0)) {
#pragma unroll
            for (int b = 0; b < kQB; ++b)
#pragma unroll
                for (int dt = 0; dt < ND; ++dt) oacc[b][dt] *= alpha[b];
        }
    };

    // O^T += V^T P^T of the block in V buffer vbuf, two 32-key chunks; step
    // i = (kc, dt), operands read one step ahead
    auto pv_product = [&](auto buf, const Vec16 (&pf)[kQB][2]) {
        typedef short v4s __attribute__((ext_vector_type(4)));
        const uint16_t* vb = vbuf(buf);
        auto fetch = [&](int i) {
            const int kc = i / ND, dt = i % ND;
            const uint16_t* a = vb + (vaddr0 ^ (16 * dt)) + 32 * D * kc;
            const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)a);
            const v4s hi =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(a + 16 * D));
            const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
            return Vec16{{l2.x, l2.y, h2.x, h2.y}};
        };
        constexpr int NS = 2 * ND;
        Vec16 va[2];
        va[0] = fetch(0);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if (i + 1 < NS) va[(i + 1) & 1] = fetch(i + 1);
            const int kc = i / ND, dt = i % ND;
#pragma unroll
            for (int b = 0; b < kQB; ++b) oacc[b][dt] = MfmaOps<T>::mma(va[i & 1], pf[b][kc], oacc[b][dt]);
        }
    };

    // ---- pipeline over the split's blocks j = 0 .. nb-1: iteration j starts
    // after a barrier that publishes K_{j+1} and V_j, issues V_{j+1} and
    // K_{j+2} into the buffers freed by the barrier, forms S_{j+1} on the
    // matrix cores while the softmax of block j runs on the vector ALUs, and
    // ends with the PV product of block j ----
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    issue_k(0, B0{});
    issue_v(0, B0{});
    if (nb > 1) {
        issue_k(1, B1{});
        __builtin_amdgcn_s_waitcnt(kWaitVm(NI));  // K_0 and V_0 (and Q) have landed
    } else {
        __builtin_amdgcn_s_waitcnt(kWaitVm(0));
    }
    __syncthreads();
    f4_t sc[kQB][4];
    s_product(B0{}, sc);
    // block j uses K buffer j & 1 and V buffer j & 1; the loop is unrolled by
    // two so every buffer choice is a compile-time constant
    auto step = [&](int j, auto par) {
        constexpr int P = decltype(par)::value;
        using Pn = std::integral_constant<int, P ^ 1>;
        __builtin_amdgcn_s_waitcnt(kWaitVm(0));
        __syncthreads();
        issue_v(j + 1, Pn{});
        if (j + 2 < nb) issue_k(j + 2, par);
        f4_t sn[kQB][4];
        Vec16 pf[kQB][2];
        float alpha[kQB];
        bool rescale = false;
        softmax(sc, pf, alpha, rescale, k_lo + j * kBN, std::false_type{});
        s_product(Pn{}, sn);
        rescale_o(alpha, rescale);
        pv_product(par, pf);
#pragma unroll
        for (int b = 0; b < kQB; ++b)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) sc[b][mt] = sn[b][mt];
    };
    for (int j = 0; j + 1 < nb; j += 2) {
        step(j, B0{});
        if (j + 2 < nb) step(j + 1, B1{});
    }
    {
        __builtin_amdgcn_s_waitcnt(kWaitVm(0));
        __syncthreads();
        const int kb = k_lo + (nb - 1) * kBN;
        Vec16 pf[kQB][2];
        float alpha[kQB];
        bool rescale = false;
        if (kb + kBN > k_hi)
            softmax(sc, pf, alpha, rescale, kb, std::true_type{});
        else
            softmax(sc, pf, alpha, rescale, kb, std::false_type{});
        rescale_o(alpha, rescale);
        if ((nb - 1) & 1)
            pv_product(B1{}, pf);
        else
            pv_product(B0{}, pf);
    }

    float l_tot[kQB];
#pragma unroll
    for (int b = 0; b < kQB; ++b) {
        l_tot[b] = col4_sum(l_run[b]);
        m_run[b] *= p.scale_log2;  // to the log2 units of the tree walk's scores
    }

    {
        // ---- partial state of this split: (m, l, acc / l).  For fp16
        // inputs the normalised numerator is stored in fp16, which halves the
        // bytes the merge reads, as the reference's own split pipelines hand
        // fp16 partial outputs to their merge (scripts/benchmark_micro.py:
        // 576-592, src/ragged_attn.py:1619); bf16 inputs keep fp32 states. ----
        const int64_t plane = p.total_tokens * (int64_t)p.Hq;
#pragma unroll
        for (int b = 0; b < kQB; ++b) {
            int64_t qrow;
            int qh;
            if (!query_of(b, qrow, qh)) continue;
            const int64_t idx = (int64_t)split * plane + qrow * p.Hq + qh;
            if (lq == 0) {
                p.part_m[idx] = m_run[b];
                p.part_l[idx] = l_tot[b];
            }
            const float inv = l_tot[b] > 0.f ? 1.f / l_tot[b] : 0.f;
            const int64_t off = idx * D + 4 * lq;
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) {
                if constexpr (kPartHalf<T>)
                    *reinterpret_cast<uint2*>((uint16_t*)p.part_acc + off + 16 * dt) =
                        make_uint2(MfmaOps<F16>::pack2(oacc[b][dt][0] * inv, oacc[b][dt][1] * inv),
                                   MfmaOps<F16>::pack2(oacc[b][dt][2] * inv, oacc[b][dt][3] * inv));
                else
                    *reinterpret_cast<float4*>((float*)p.part_acc + off + 16 * dt) =
                        make_float4(oacc[b][dt][0] * inv, oacc[b][dt][1] * inv, oacc[b][dt][2] * inv,
                                    oacc[b][dt][3] * inv);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Split merge of the prefix-only pass: 4 lanes per (token, q head) fold the
// splits' partial states and store the normalised output (+ LSE).
// ---------------------------------------------------------------------------
// TPB: threads per workgroup (one wave when 256-thread workgroups would
// occupy under half the CUs: four times the CUs then share the loads).
template <typename T, int D, bool LSE, bool BATCH, int TPB = kPrefixThreads>
__global__ __launch_bounds__(kPrefixThreads) void prefix_merge_kernel(TreeParams p) {
    constexpr int SLOTS = TPB / 4;
    const int j = threadIdx.x & 3;
    const int64_t slot = (int64_t)blockIdx.x * SLOTS + (threadIdx.x >> 2);
    int h, tok, seq;
    slot_coords(p, slot, (int64_t)gridDim.x * SLOTS, h, tok, seq);
    if (seq >= p.B) return;
    int32_t start, n;
    if (!seq_bounds<BATCH>(p, seq, start, n)) return;
    if (tok >= n) return;
    const int64_t qrow = (int64_t)start + tok;
    float m, l, acc[8 * (D / 32)];
    load_partial_state4<T, D>(p, qrow, h, j, m, l, acc);
    write_out4<T, D, LSE, BATCH>(p, seq, qrow, h, j, m, l, acc);
}

template <typename T, int D, bool BATCH>
static int launch_prefix_merge(const TreeParams& p, hipStream_t st) {
    constexpr int SLOTS = kPrefixThreads / 4;
    const int64_t blocks = ((int64_t)p.B * p.max_seqlen * p.Hq + SLOTS - 1) / SLOTS;
    if (blocks >= (int64_t(1) << 31)) {
        set_error("merge grid too large (%lld blocks)", (long long)blocks);
        return QATTN_ERR_ARG;
    }
    const dim3 g((unsigned)blocks), b(kPrefixThreads);
    const bool small = blocks < 128;  // under half the CUs: one-wave workgroups instead
    const dim3 g1((unsigned)(blocks * (kPrefixThreads / 64))), b1(64);
    if (p.lse && small)
        hipLaunchKernelGGL((prefix_merge_kernel<T, D, true, BATCH, 64>), g1, b1, 0, st, p);
    else if (p.lse)
        hipLaunchKernelGGL((prefix_merge_kernel<T, D, true, BATCH>), g, b, 0, st, p);
    else if (small)
        hipLaunchKernelGGL((prefix_merge_kernel<T, D, false, BATCH, 64>), g1, b1, 0, st, p);
    else
        hipLaunchKernelGGL((prefix_merge_kernel<T, D, false, BATCH>), g, b, 0, st, p);
    return launch_status("prefix_merge_kernel");
}

template <typename T>
static int run_prefix_merge(const TreeParams& p, int head_dim, hipStream_t st) {
    if (!p.cu) {
        return head_dim == 32   ? launch_prefix_merge<T, 32, true>(p, st)
               : head_dim == 64 ? launch_prefix_merge<T, 64, true>(p, st)
                                : launch_prefix_merge<T, 128, true>(p, st);
    }
    return head_dim == 32   ? launch_prefix_merge<T, 32, false>(p, st)
           : head_dim == 64 ? launch_prefix_merge<T, 64, false>(p, st)
                            : launch_prefix_merge<T, 128, false>(p, st);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int64_t units_per_split(int batch, int hkv, int max_seqlen, int group, int bm = kBM) {
    const int64_t qtiles = ((int64_t)max_seqlen * group + bm - 1) / bm;
    return (int64_t)batch * hkv * qtiles;
}

// Split count along the prefix: enough work units for ~2 resident workgroups
// on each of 256 CUs, never more splits than 64-key blocks.
static int prefix_splits(int64_t ups, int L, int num_splits, int& blocks_per_split) {
    const int blocks = (L + kBN - 1) / kBN;
    int s = num_splits;
    if (s <= 0) {
        s = (int)std::max<int64_t>(1, (512 + ups / 2) / ups);
        // Every split writes a partial state that the merge reads back; with
        // few query rows (one decode step of a small tree) that traffic and the
        // per-split overheads outgrow the split's own work.  Keep at least an
        // eighth of the blocks, within 2..8, per split (one EAGLE-3 step over
        // a 2048-token cache runs 17.2 us per call with 8 splits, 18.8 with 4,
        // 21.5 with 16).
        const int bps_min = std::min(8, std::max(2, blocks / 8));
        s = std::min(s, std::max(1, blocks / bps_min));
    }
    s = std::max(1, std::min(s, std::max(blocks, 1)));
    blocks_per_split = (blocks + s - 1) / s;
    return blocks_per_split > 0 ? (blocks + blocks_per_split - 1) / blocks_per_split : 1;
}

static int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// Split-state bytes: m and l in fp32, the numerator in fp16 for fp16 inputs
// (half_acc, kPartHalf) and fp32 otherwise.  qattn_prefix_workspace_bytes,
// which takes no dtype, reports the fp32 size, an upper bound for both.
static int64_t workspace_bytes(int64_t total_tokens, int hq, int head_dim, int splits, bool half_acc = false) {
    if (splits <= 1) return 0;  // one split: fused epilogue, no partial states
    const int64_t plane = total_tokens * hq;
    return 2 * align256(splits * plane * 4) + align256(splits * plane * head_dim * (half_acc ? 2 : 4));
}

template <typename T, int D, bool BATCH>
static void launch_prefix_b(const PrefixParams& pp, const TreeParams& tp, bool fused, bool half, int walk, dim3 g,
                            hipStream_t st) {
    const dim3 b(kPrefixThreads);
    if constexpr (!BATCH) {
        // walk export of the fused epilogue (the caller has checked: packed cu_seqlens)
        if (fused && tp.dbg_walk && (walk == WALK_HEAP || walk == WALK_PARENTS)) {
            if (walk == WALK_HEAP && tp.lse)
                hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, true, WALK_HEAP, false, true>), g, b, 0, st, pp,
                                   tp);
            else if (walk == WALK_HEAP)
                hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, false, WALK_HEAP, false, true>), g, b, 0, st, pp,
                                   tp);
            else if (tp.lse)
                hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, true, WALK_PARENTS, false, true>), g, b, 0, st,
                                   pp, tp);
            else
                hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, false, WALK_PARENTS, false, true>), g, b, 0, st,
                                   pp, tp);
            return;
        }
    }
    if (!fused && half)
        hipLaunchKernelGGL((prefix_half_kernel<T, D, BATCH>), g, b, 0, st, pp);
    else if (!fused)
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, false, false, WALK_HEAP, BATCH>), g, b, 0, st, pp, tp);
    else if (walk == WALK_NONE && tp.lse)
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, true, WALK_NONE, BATCH>), g, b, 0, st, pp, tp);
    else if (walk == WALK_NONE)
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, false, WALK_NONE, BATCH>), g, b, 0, st, pp, tp);
    else if (walk == WALK_PARENTS && tp.lse)
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, true, WALK_PARENTS, BATCH>), g, b, 0, st, pp, tp);
    else if (walk == WALK_PARENTS)
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, false, WALK_PARENTS, BATCH>), g, b, 0, st, pp, tp);
    else if (tp.lse)
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, true, WALK_HEAP, BATCH>), g, b, 0, st, pp, tp);
    else
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, false, WALK_HEAP, BATCH>), g, b, 0, st, pp, tp);
}

template <typename T, int D>
static int launch_prefix(const PrefixParams& pp, const TreeParams& tp, bool fused, bool half, int walk,
                         hipStream_t st) {
    const int64_t grid = ((int64_t)pp.n_units + 7) / 8 * 8;
    if (grid >= (int64_t(1) << 31)) {
        set_error("prefix grid too large");
        return QATTN_ERR_ARG;
    }
    // (a null cu is a uniform batch: its addressing is compiled separately)
    if (pp.cu)
        launch_prefix_b<T, D, false>(pp, tp, fused, half, walk, dim3((unsigned)grid), st);
    else
        launch_prefix_b<T, D, true>(pp, tp, fused, half, walk, dim3((unsigned)grid), st);
    return launch_status("prefix_attn_kernel");
}

}  // namespace qattn

using namespace qattn;

// Per-sequence offsets of a uniform batch of [B, H, N, D] views (no cu):
// element offsets added to every q / o / lse row of sequence s (times s), and
// the distance between the sequences' parent arrays.
struct BatchView {
    int64_t q_b, o_b, lse_b;
    int32_t par_stride;
};

// Shared body of the prefix entry points.  walk: WALK_HEAP walks the heap
// tree of branching_factor, WALK_PARENTS the explicit parent array,
// WALK_NONE attends the prefix only (k, v unused); bv null is the cu-packed
// layout, else a uniform batch (cu_seqlens unused).
static int prefix_tree_impl(const void* q, const int64_t q_stride[3], const void* k, const int64_t k_stride[3],
                            const void* v, const int64_t v_stride[3], const void* k_prefix,
                            const int64_t kp_stride[3], const void* v_prefix, const int64_t vp_stride[3],
                            int32_t prefix_len, void* o, const int64_t o_stride[3], float* lse,
                            const int64_t lse_stride[2], const int32_t* cu_seqlens, const int32_t* parents,
                            int32_t batch, int32_t max_seqlen, int64_t total_tokens, int64_t tree_seq_stride,
                            int64_t tree_row0, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                            int32_t branching_factor, int32_t max_depth, float scale, int32_t dtype,
                            void* workspace, int64_t workspace_size, int32_t num_splits, void* stream,
                            const BatchView* bv, int walk) {
    int rc = check_common(dtype, head_dim, batch, max_seqlen, total_tokens, num_q_heads, num_kv_heads, max_depth);
    if (rc) return rc;
    if (!(scale > 0.f)) {
        set_error("scale must be positive (got %g)", (double)scale);
        return QATTN_ERR_ARG;
    }
    if (prefix_len < 0 || tree_seq_stride < 0 || tree_row0 < 0) {
        set_error("bad prefix_len / tree layout (%d, %lld, %lld)", prefix_len, (long long)tree_seq_stride,
                  (long long)tree_row0);
        return QATTN_ERR_ARG;
    }
    if (walk == WALK_NONE && prefix_len < 1) {
        set_error("prefix-only attention needs prefix_len >= 1 (got %d)", prefix_len);
        return QATTN_ERR_ARG;
    }
    if (batch == 0 || max_seqlen == 0 || total_tokens == 0) return QATTN_OK;
    // (the prefix-only pass reads no tree rows: q stands in for k and v)
    const bool tree = walk != WALK_NONE;
    TreeParams tp;
    rc = fill_tree_params(tp, q, q_stride, tree ? k : q, tree ? k_stride : q_stride, tree ? v : q,
                          tree ? v_stride : q_stride, o, o_stride, lse, lse_stride, cu_seqlens, batch, max_seqlen,
                          total_tokens, num_q_heads, num_kv_heads, branching_factor, max_depth, scale,
                          bv != nullptr);
    if (rc) return rc;
    if (bv) {
        tp.cu = nullptr;
        tp.sq_b = bv->q_b;
        tp.so_b = bv->o_b;
        tp.slse_b = bv->lse_b;
        tp.par_stride = bv->par_stride;
    }
    if (tree && (!row_aligned(k, k_stride, 2) || !row_aligned(v, v_stride, 2))) {
        set_error("k/v rows must be 16-byte aligned with stride_dim 1");
        return QATTN_ERR_LAYOUT;
    }
    tp.kv_seq_stride = tree_seq_stride;
    tp.kv_row0 = tree_row0;
    tp.parents = parents;
    hipStream_t st = (hipStream_t)stream;
    if (prefix_len == 0) return run_tree(tp, dtype, head_dim, walk, KV_PACKED, false, QATTN_ALGO_AUTO, st);

    if (!k_prefix || !v_prefix || !kp_stride || !vp_stride) {
        set_error("prefix pointers are null");
        return QATTN_ERR_ARG;
    }
    if (((uintptr_t)k_prefix & 15) || ((uintptr_t)v_prefix & 15) || kp_stride[1] % 8 || kp_stride[2] % 8 ||
        vp_stride[1] % 8 || vp_stride[2] % 8 || kp_stride[0] % 8 || vp_stride[0] % 8) {
        set_error("prefix rows must be 16-byte aligned (strides in multiples of 8 elements)");
        return QATTN_ERR_LAYOUT;
    }
    // the kernel addresses a 64-key block with 32-bit byte offsets
    if (kp_stride[1] < 0 || vp_stride[1] < 0 ||
        (int64_t)kBN * std::max(kp_stride[1], vp_stride[1]) * 2 >= (int64_t(1) << 32)) {
        set_error("prefix token strides must be non-negative and below 2^25 elements");
        return QATTN_ERR_LAYOUT;
    }
    const int g = num_q_heads / num_kv_heads;
    int bps = 0;
    const int64_t ups = units_per_split(batch, num_kv_heads, max_seqlen, g);
    const int splits = prefix_splits(ups, prefix_len, num_splits, bps);
    const int64_t need = workspace_bytes(total_tokens, num_q_heads, head_dim, splits, dtype == QATTN_DTYPE_F16);
    if (need > 0 && (!workspace || workspace_size < need || ((uintptr_t)workspace & 255))) {
        set_error("workspace of %lld bytes (256-byte aligned) required, got %lld", (long long)need,
                  (long long)workspace_size);
        return QATTN_ERR_WORKSPACE;
    }
    if (ups * splits >= (int64_t(1) << 31)) {
        set_error("too many prefix work units");
        return QATTN_ERR_ARG;
    }
    const bool fused = splits == 1;
    if (tp.dbg_walk && !tp.cu) {
        set_error("the walk export runs calls over packed cu_seqlens");
        return QATTN_ERR_ARG;
    }
    const int64_t plane = total_tokens * num_q_heads;
    PrefixParams pp{};
    pp.q = q;
    pp.kp = k_prefix;
    pp.vp = v_prefix;
    pp.cu = tp.cu;
    if (!fused) {
        pp.part_m = (float*)workspace;
        pp.part_l = (float*)((char*)workspace + align256(splits * plane * 4));
        pp.part_acc = (char*)workspace + 2 * align256(splits * plane * 4);
    }
    pp.sq_t = q_stride[0];
    pp.sq_h = q_stride[1];
    pp.sq_b = tp.sq_b;
    pp.skp_b = kp_stride[0];
    pp.skp_t = kp_stride[1];
    pp.skp_h = kp_stride[2];
    pp.svp_b = vp_stride[0];
    pp.svp_t = vp_stride[1];
    pp.svp_h = vp_stride[2];
    pp.total_tokens = total_tokens;
    pp.B = batch;
    pp.Hq = num_q_heads;
    pp.Hkv = num_kv_heads;
    pp.group = g;
    pp.max_seqlen = max_seqlen;
    pp.L = prefix_len;
    pp.n_split = splits;
    pp.blocks_per_split = bps;
    // Split units that would leave CUs idle (fewer than one per CU: a decode
    // step of a small tree) take half-height query tiles, twice as many.
    const bool half = !fused && ups * splits < 256;
    const int bm = half ? kBM / 2 : kBM;
    pp.qtiles = (int32_t)(((int64_t)max_seqlen * g + bm - 1) / bm);
    pp.n_units = (int32_t)(units_per_split(batch, num_kv_heads, max_seqlen, g, bm) * splits);
    pp.gdiv = make_divider(g);
    pp.qtdiv = make_divider(pp.qtiles);
    pp.nsdiv = make_divider(splits);
    pp.hkvdiv = make_divider(num_kv_heads);
    pp.scale_log2 = scale * kLog2e;
    if (dtype == QATTN_DTYPE_F16) {
        rc = head_dim == 32   ? launch_prefix<F16, 32>(pp, tp, fused, half, walk, st)
             : head_dim == 64 ? launch_prefix<F16, 64>(pp, tp, fused, half, walk, st)
                              : launch_prefix<F16, 128>(pp, tp, fused, half, walk, st);
    } else {
        rc = head_dim == 32   ? launch_prefix<BF16, 32>(pp, tp, fused, half, walk, st)
             : head_dim == 64 ? launch_prefix<BF16, 64>(pp, tp, fused, half, walk, st)
                              : launch_prefix<BF16, 128>(pp, tp, fused, half, walk, st);
    }
    if (rc || fused) return rc;
    tp.part_m = pp.part_m;
    tp.part_l = pp.part_l;
    tp.part_acc = pp.part_acc;
    tp.n_split = splits;
    if (!tree)
        return dtype == QATTN_DTYPE_F16 ? run_prefix_merge<F16>(tp, head_dim, st)
                                        : run_prefix_merge<BF16>(tp, head_dim, st);
    return run_tree(tp, dtype, head_dim, walk, KV_PACKED, true, QATTN_ALGO_AUTO, st);
}

// The [B, H, N, D] view entry (qattn_ragged_tree_attn_fwd and its
// allocation-free variant): strides to the packed form, then prefix_tree_impl.
static int ragged_tree_attn_impl(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                                 const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4],
                                 float* lse, const int64_t lse_stride[3], const int32_t* parents,
                                 int64_t parents_stride, int32_t batch, int32_t num_tree, int32_t num_prefix,
                                 int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                 int32_t branching_factor, int32_t max_depth, float scale, int32_t dtype,
                                 void* workspace, int64_t workspace_size, int32_t num_splits, void* stream) {
    if (!q_stride || !k_stride || !v_stride || !o_stride || (lse && !lse_stride)) {
        set_error("null stride array");
        return QATTN_ERR_ARG;
    }
    const int64_t total = (int64_t)batch * num_tree;
    int rc = check_common(dtype, head_dim, batch, num_tree, total, num_q_heads, num_kv_heads, max_depth);
    if (rc) return rc;
    if (num_prefix < 0 || parents_stride < 0) {
        set_error("bad num_prefix / parents_stride (%d, %lld)", num_prefix, (long long)parents_stride);
        return QATTN_ERR_ARG;
    }
    if (batch == 0 || num_tree == 0) return QATTN_OK;
    // (token, head, dim) strides of each tensor; a batch stride only matters
    // when there is more than one sequence
    const int64_t q3[3] = {q_stride[2], q_stride[1], q_stride[3]};
    const int64_t o3[3] = {o_stride[2], o_stride[1], o_stride[3]};
    const int64_t k3[3] = {k_stride[2], k_stride[1], k_stride[3]};
    const int64_t v3[3] = {v_stride[2], v_stride[1], v_stride[3]};
    const bool many = batch > 1;
    const int64_t qb = many ? q_stride[0] : 0, ob = many ? o_stride[0] : 0;
    const int64_t kb = many ? k_stride[0] : 0, vb = many ? v_stride[0] : 0;
    if (qb % 8 || ob % 8) {
        set_error("q/o batch strides must keep rows 16-byte aligned (multiples of 8 elements)");
        return QATTN_ERR_LAYOUT;
    }
    // tree row n of sequence s is k/v row s * seq_rows + num_prefix + n
    int64_t seq_rows = 1;  // one sequence: any non-zero value
    if (many) {
        if (kb <= 0 || k3[0] <= 0 || v3[0] <= 0 || kb % k3[0] || vb % v3[0] || kb / k3[0] != vb / v3[0]) {
            set_error("k/v batch strides must be the same positive multiple of their token strides");
            return QATTN_ERR_LAYOUT;
        }
        seq_rows = kb / k3[0];
    }
    if (parents && (int64_t)(batch - 1) * (many ? parents_stride : 0) + num_tree > INT32_MAX) {
        set_error("parent array too large");
        return QATTN_ERR_ARG;
    }
    BatchView bv;
    bv.q_b = many ? qb - num_tree * q3[0] : 0;
    bv.o_b = many ? ob - num_tree * o3[0] : 0;
    bv.lse_b = lse && many ? lse_stride[0] - num_tree * lse_stride[2] : 0;
    bv.par_stride = many ? (int32_t)parents_stride : 0;
    const int64_t lse2[2] = {lse ? lse_stride[2] : 0, lse ? lse_stride[1] : 0};
    // the prefix is rows 0 .. num_prefix - 1 of every sequence's k/v
    const int64_t kp3[3] = {kb, k3[0], k3[1]};
    const int64_t vp3[3] = {vb, v3[0], v3[1]};
    return prefix_tree_impl(q, q3, k, k3, v, v3, k, kp3, v, vp3, num_prefix, o, o3, lse, lse ? lse2 : nullptr,
                            nullptr, parents, batch, num_tree, total, seq_rows, num_prefix, num_q_heads,
                            num_kv_heads, head_dim, parents ? 1 : branching_factor, max_depth, scale, dtype,
                            workspace, workspace_size, num_splits, stream, &bv,
                            parents ? WALK_PARENTS : WALK_HEAP);
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point: a static device array (each GPU
// the library runs on holds its own copy until the process ends).  Host code
// never passes `scratch` itself to a kernel (on the host it is only a
// stand-in for the symbol): it uses the device address from
// hipGetSymbolAddress, kept per device.
// ---------------------------------------------------------------------------
constexpr int64_t kScratchBytes = int64_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kScratchMaxDev = 64;
std::mutex g_scratch_mu;
void* g_scratch[kScratchMaxDev] = {};
}  // namespace

// Device address of the current device's scratch (hipGetSymbolAddress once
// per device, with that device current), or null with the error set.
static void* scratch_ptr() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchMaxDev) {
        set_error("no usable current device (%d) for the scratch array", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            set_error("hipGetSymbolAddress(scratch) failed on device %d", dev);
            return nullptr;
        }
        g_scratch[dev] = ptr;
    }
    return g_scratch[dev];
}

extern "C" {

int qattn_init(void) {
    clear_error();
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        set_error("hipGetDevice failed");
        return QATTN_ERR_HIP;
    }
    const int rc = sched_init(dev);
    if (rc) return rc;
    return scratch_ptr() ? QATTN_OK : QATTN_ERR_HIP;
}

int qattn_sched_info(int64_t info[6]) {
    clear_error();
    if (!info) {
        set_error("info is null");
        return QATTN_ERR_ARG;
    }
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        set_error("hipGetDevice failed");
        return QATTN_ERR_HIP;
    }
    return sched_info(dev, info);
}

int64_t qattn_prefix_workspace_bytes(int32_t batch, int32_t max_seqlen, int64_t total_tokens, int32_t num_q_heads,
                                     int32_t num_kv_heads, int32_t head_dim, int32_t prefix_len, int32_t num_splits) {
    if (batch <= 0 || max_seqlen <= 0 || total_tokens <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
        num_q_heads % num_kv_heads || prefix_len <= 0)
        return 0;
    int bps = 0;
    const int splits =
        prefix_splits(units_per_split(batch, num_kv_heads, max_seqlen, num_q_heads / num_kv_heads), prefix_len,
                      num_splits, bps);
    return workspace_bytes(total_tokens, num_q_heads, head_dim, splits);
}

int qattn_prefix_tree_fwd(const void* q, const int64_t q_stride[3], const void* k, const int64_t k_stride[3],
                          const void* v, const int64_t v_stride[3], const void* k_prefix,
                          const int64_t kp_stride[3], const void* v_prefix, const int64_t vp_stride[3],
                          int32_t prefix_len, void* o, const int64_t o_stride[3], float* lse,
                          const int64_t lse_stride[2], const int32_t* cu_seqlens, int32_t batch,
                          int32_t max_seqlen, int64_t total_tokens, int64_t tree_seq_stride, int64_t tree_row0,
                          int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t branching_factor,
                          int32_t max_depth, float scale, int32_t dtype, void* workspace, int64_t workspace_size,
                          int32_t num_splits, void* stream) {
    clear_error();
    return prefix_tree_impl(q, q_stride, k, k_stride, v, v_stride, k_prefix, kp_stride, v_prefix, vp_stride,
                            prefix_len, o, o_stride, lse, lse_stride, cu_seqlens, nullptr, batch, max_seqlen,
                            total_tokens, tree_seq_stride, tree_row0, num_q_heads, num_kv_heads, head_dim,
                            branching_factor, max_depth, scale, dtype, workspace, workspace_size, num_splits, stream,
                            nullptr, WALK_HEAP);
}

int qattn_prefix_tree_parents_fwd(const void* q, const int64_t q_stride[3], const void* k,
                                  const int64_t k_stride[3], const void* v, const int64_t v_stride[3],
                                  const void* k_prefix, const int64_t kp_stride[3], const void* v_prefix,
                                  const int64_t vp_stride[3], int32_t prefix_len, void* o,
                                  const int64_t o_stride[3], float* lse, const int64_t lse_stride[2],
                                  const int32_t* cu_seqlens, const int32_t* parents, int32_t batch,
                                  int32_t max_seqlen, int64_t total_tokens, int64_t tree_seq_stride,
                                  int64_t tree_row0, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t max_depth, float scale, int32_t dtype, void* workspace,
                                  int64_t workspace_size, int32_t num_splits, void* stream) {
    clear_error();
    if (!parents && batch > 0 && max_seqlen > 0 && total_tokens > 0) {
        set_error("parents is null");
        return QATTN_ERR_ARG;
    }
    return prefix_tree_impl(q, q_stride, k, k_stride, v, v_stride, k_prefix, kp_stride, v_prefix, vp_stride,
                            prefix_len, o, o_stride, lse, lse_stride, cu_seqlens, parents, batch, max_seqlen,
                            total_tokens, tree_seq_stride, tree_row0, num_q_heads, num_kv_heads, head_dim, 1,
                            max_depth, scale, dtype, workspace, workspace_size, num_splits, stream, nullptr,
                            WALK_PARENTS);
}

int qattn_prefix_fwd(const void* q, const int64_t q_stride[3], const void* k_prefix, const int64_t kp_stride[3],
                     const void* v_prefix, const int64_t vp_stride[3], int32_t prefix_len, void* o,
                     const int64_t o_stride[3], float* lse, const int64_t lse_stride[2],
                     const int32_t* cu_seqlens, int32_t batch, int32_t max_seqlen, int64_t total_tokens,
                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float scale, int32_t dtype,
                     void* workspace, int64_t workspace_size, int32_t num_splits, void* stream) {
    clear_error();
    return prefix_tree_impl(q, q_stride, nullptr, nullptr, nullptr, nullptr, k_prefix, kp_stride, v_prefix,
                            vp_stride, prefix_len, o, o_stride, lse, lse_stride, cu_seqlens, nullptr, batch,
                            max_seqlen, total_tokens, 0, 0, num_q_heads, num_kv_heads, head_dim, 1, 0, scale, dtype,
                            workspace, workspace_size, num_splits, stream, nullptr, WALK_NONE);
}

int qattn_ragged_tree_attn_fwd(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                               const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4],
                               float* lse, const int64_t lse_stride[3], const int32_t* parents,
                               int64_t parents_stride, int32_t batch, int32_t num_tree, int32_t num_prefix,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t branching_factor, int32_t max_depth, float scale, int32_t dtype,
                               void* workspace, int64_t workspace_size, int32_t num_splits, void* stream) {
    clear_error();
    return ragged_tree_attn_impl(q, q_stride, k, k_stride, v, v_stride, o, o_stride, lse, lse_stride, parents,
                                 parents_stride, batch, num_tree, num_prefix, num_q_heads, num_kv_heads, head_dim,
                                 branching_factor, max_depth, scale, dtype, workspace, workspace_size, num_splits,
                                 stream);
}

int qattn_ragged_tree_attn_fwd_noalloc(const void* q, const int64_t q_stride[4], const void* k,
                                       const int64_t k_stride[4], const void* v, const int64_t v_stride[4], void* o,
                                       const int64_t o_stride[4], float* lse, const int64_t lse_stride[3],
                                       const int32_t* parents, int64_t parents_stride, int32_t batch,
                                       int32_t num_tree, int32_t num_prefix, int32_t num_q_heads,
                                       int32_t num_kv_heads, int32_t head_dim, int32_t branching_factor,
                                       int32_t max_depth, float scale, int32_t dtype, int32_t num_splits,
                                       void* stream) {
    clear_error();
    if (batch > 0 && num_tree > 0 && num_prefix > 0 && num_q_heads > 0 && num_kv_heads > 0 &&
        num_q_heads % num_kv_heads == 0 && num_splits >= 0) {
        // the split states must fit the scratch array: the automatic count
        // drops to the largest that fits (one split needs none), an explicit
        // one that does not fit is an error
        const int64_t total = (int64_t)batch * num_tree;
        const int64_t ups = units_per_split(batch, num_kv_heads, num_tree, num_q_heads / num_kv_heads);
        int bps = 0;
        int s = prefix_splits(ups, num_prefix, num_splits, bps);
        const bool half = dtype == QATTN_DTYPE_F16;  // fp16 split numerators (kPartHalf)
        if (workspace_bytes(total, num_q_heads, head_dim, s, half) > kScratchBytes) {
            if (num_splits > 0) {
                set_error("%d prefix splits need %lld bytes of split state; the scratch array holds %lld", s,
                          (long long)workspace_bytes(total, num_q_heads, head_dim, s, half),
                          (long long)kScratchBytes);
                return QATTN_ERR_WORKSPACE;
            }
            while (s > 1 && workspace_bytes(total, num_q_heads, head_dim, s, half) > kScratchBytes) --s;
            num_splits = s;
        }
    }
    void* ws = scratch_ptr();
    if (!ws) return QATTN_ERR_HIP;
    return ragged_tree_attn_impl(q, q_stride, k, k_stride, v, v_stride, o, o_stride, lse, lse_stride, parents,
                                 parents_stride, batch, num_tree, num_prefix, num_q_heads, num_kv_heads, head_dim,
                                 branching_factor, max_depth, scale, dtype, ws, kScratchBytes, num_splits, stream);
}

}  // extern "C"
