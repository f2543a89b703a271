// tree_walk.h -- device-side pieces of the ancestor walk shared by the tree
// kernels (tree_attn.hip) and the fused epilogue of the prefix kernel
// (prefix_attn.hip).
//
// A query (token, q head) is owned by a group of 4 consecutive lanes; lane j
// holds the 16-byte chunks j, j+4, j+8, ... of every D-element head row (Q, K,
// V rows and the fp32 accumulator), so a chunk of the row is 64 contiguous
// bytes per group and the dot-product reduction is a 2-step DPP quad sum.
// Scores are kept in the log2 domain: s = (q . k) * scale * log2(e).
#pragma once

#include "qattn_common.h"
#include "qattn_device.h"

namespace qattn {

// WALK_NONE: no tree keys (the prefix-only pass of the prefix kernel)
enum { WALK_HEAP = 0, WALK_PARENTS = 1, WALK_NONE = 2 };
enum { KV_PACKED = 0, KV_PAGED = 1 };

__device__ __forceinline__ int rl(int v, int i) { return __builtin_amdgcn_readlane(v, i); }

// Sequence bounds with the guards documented in qattn.h.
// BATCH (a uniform batch, null cu): sequence seq holds rows
// [seq * max_seqlen, (seq + 1) * max_seqlen).
template <bool BATCH = false>
__device__ __forceinline__ bool seq_bounds(const TreeParams& p, int seq, int32_t& start, int32_t& n) {
    if constexpr (BATCH) {
        start = seq * p.max_seqlen;
        n = p.max_seqlen;
        return true;
    }
    int32_t s = p.cu[seq], e = p.cu[seq + 1];
    if (s < 0 || e < s || (int64_t)e > p.total_tokens) return false;
    start = s;
    n = e - s;
    if (n > p.max_seqlen) n = p.max_seqlen;
    return true;
}

// First tree K/V row of a sequence: cu-packed, or the hybrid layout where each
// sequence's tree rows follow its prefix rows.
__device__ __forceinline__ int64_t kv_base(const TreeParams& p, int seq, int32_t start) {
    return p.kv_seq_stride ? (int64_t)seq * p.kv_seq_stride + p.kv_row0 : (int64_t)start;
}

// Index of a sequence's first entry in the parent array: its first row
// (packed by cu), or seq * par_stride (uniform batch; stride 0 shares one
// array between all sequences).
template <bool BATCH = false>
__device__ __forceinline__ int32_t parents_base(const TreeParams& p, int seq, int32_t start) {
    return BATCH ? seq * p.par_stride : start;
}

// Next node of the walk (src/ragged_attn.py:376-377 heap, :692-694 parents);
// pb is the sequence's parents_base.
template <int WALK>
__device__ __forceinline__ int32_t walk_next(const TreeParams& p, int32_t pb, int32_t n, int32_t cur) {
    if constexpr (WALK == WALK_HEAP) {
        return heap_parent(cur, p.bdiv);
    } else {
        const int32_t par = p.parents[pb + cur];
        return (par >= 0 && par < n) ? par : cur;
    }
}

// A (token, q head) slot of the 4-lanes-per-query kernels (q head fastest)
// as q head, token and sequence: 32-bit magic-number divisions (the 64-bit
// divisions held a small launch's first loads back by ~0.5 us) whenever the
// grid's slots fit in 31 bits (wave-uniform), else 64-bit.
__device__ __forceinline__ void slot_coords(const TreeParams& p, int64_t slot, int64_t nslots, int& h, int& tok,
                                            int& seq) {
    if (nslots < (int64_t(1) << 31)) {
        const int32_t s32 = (int32_t)slot;
        const int32_t r = divide(s32, p.hqdiv);
        h = s32 - r * p.Hq;
        seq = divide(r, p.msdiv);
        tok = r - seq * p.max_seqlen;
    } else {
        h = (int)(slot % p.Hq);
        const int64_t rest = slot / p.Hq;
        tok = (int)(rest % p.max_seqlen);
        seq = (int)(rest / p.max_seqlen);
    }
}

// Q fragment of a query in the 4-lane layout.
template <int D, bool BATCH = false>
__device__ __forceinline__ void load_q4(const TreeParams& p, int seq, int64_t qrow, int h, int j, Vec16* qf) {
    const uint16_t* qp = (const uint16_t*)p.q + qrow * p.sq_t + (BATCH ? (int64_t)seq * p.sq_b : 0) +
                         (int64_t)h * p.sq_h + 8 * j;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) qf[i] = ld16(qp + 32 * i);
}

// Initial state from split-K prefix partials (flash-decoding merge of all
// splits): m = max_s m_s, w_s = 2^(m_s - m) l_s, l = sum_s w_s and acc =
// sum_s w_s a_s, a_s being split s's numerator / l_s as stored (fp16 for
// fp16 inputs, else fp32: see kPartHalf).  The splits
// are folded in batches of SP whose loads are issued together, each batch
// moving the running maximum once (an online merge: no separate pass for the
// maxima), so n splits cost about n / SP memory round trips.
template <typename T, int D>
__device__ __forceinline__ void load_partial_state4(const TreeParams& p, int64_t qrow, int h, int j,
                                                    float& m, float& l, float* acc) {
    constexpr int NCH = D / 32;
    constexpr bool H = kPartHalf<T>;
    constexpr int W = H ? 1 : 2;  // 16-byte loads per 8-element chunk
    // splits per batch: 4 (fp16 states) or 3 (fp32) at head_dim 128; 6 fp16
    // states per batch needed more than 256 VGPRs in the gather kernel
    constexpr int SP = (H && NCH == 4) ? 4 : 12 / NCH;
    const int ns = p.n_split;
    const int64_t plane = p.total_tokens * (int64_t)p.Hq;
    const int64_t idx = qrow * p.Hq + h;
    m = -INFINITY;
    l = 0.f;
#pragma unroll
    for (int e = 0; e < 8 * NCH; ++e) acc[e] = 0.f;
    for (int s0 = 0; s0 < ns; s0 += SP) {
        float ms[SP], ls[SP];
        Vec16 a[SP][W * NCH];  // numerator / l of split s0 + u, 8 elements per chunk
#pragma unroll
        for (int u = 0; u < SP; ++u) {
            ms[u] = -INFINITY;
            ls[u] = 0.f;
#pragma unroll
            for (int i = 0; i < W * NCH; ++i) a[u][i] = Vec16{{0u, 0u, 0u, 0u}};
            if (s0 + u < ns) {  // wave-uniform
                const int64_t k = (s0 + u) * plane + idx;
                ms[u] = p.part_m[k];
                ls[u] = p.part_l[k];
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    if constexpr (H) {
                        a[u][i] = ld16((const uint16_t*)p.part_acc + k * D + 8 * j + 32 * i);
                    } else {
                        const float* src = (const float*)p.part_acc + k * D + 8 * j + 32 * i;
                        a[u][2 * i] = ld16(src);
                        a[u][2 * i + 1] = ld16(src + 4);
                    }
                }
            }
        }
        float mb = m;
#pragma unroll
        for (int u = 0; u < SP; ++u) mb = fmaxf(mb, ms[u]);
        if (mb == -INFINITY) continue;  // nothing attended so far
        if (m != -INFINITY && mb != m) {
            const float alpha = fast_exp2(m - mb);
            l *= alpha;
#pragma unroll
            for (int e = 0; e < 8 * NCH; ++e) acc[e] *= alpha;
        }
        m = mb;
#pragma unroll
        for (int u = 0; u < SP; ++u) {
            const float w = ms[u] == -INFINITY ? 0.f : fast_exp2(ms[u] - m);
            const float wl = w * ls[u];  // weight of the normalised numerator
            l += wl;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                float* c = acc + 8 * i;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = H ? ((e & 1) ? MfmaOps<F16>::hi(a[u][i].w[e >> 1])
                                                 : MfmaOps<F16>::lo(a[u][i].w[e >> 1]))
                                      : __builtin_bit_cast(float, a[u][2 * i + (e >> 2)].w[e & 3]);
                    c[e] = __builtin_fmaf(wl, x, c[e]);
                }
            }
        }
    }
}

// Partial dot product of the lane's chunks, reduced over the 4-lane group.
template <typename T, int NCH>
__device__ __forceinline__ float qk4(const Vec16* qf, const Vec16* kf) {
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) d += dot8<T>(qf[i], kf[i]);
    return group_sum<4>(d);
}

// Merge NS scores (log2 domain, -inf = not attended) and their V fragments
// into (m, l, acc): one max, one rescale, NS exponentials.
template <typename T, int NCH, int NS>
__device__ __forceinline__ void fold_scores(const float* s, const Vec16 (*vf)[NCH], float& m, float& l,
                                            float* acc) {
    float cm = s[0];
#pragma unroll
    for (int t = 1; t < NS; ++t) cm = fmaxf(cm, s[t]);
    const float m_new = fmaxf(m, cm);
    if (m_new == -INFINITY) return;  // nothing attended yet
    if (m != -INFINITY) {
        const float alpha = fast_exp2(m - m_new);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < 8 * NCH; ++e) acc[e] *= alpha;
    }
#pragma unroll
    for (int t = 0; t < NS; ++t) {
        const float pt = fast_exp2(s[t] - m_new);  // exp2(-inf) = 0 for skipped steps
        l += pt;
#pragma unroll
        for (int i = 0; i < NCH; ++i) axpy8<T>(acc + 8 * i, pt, vf[t][i]);
    }
    m = m_new;
}

// The ancestor walk of one query with K/V rows gathered from global memory:
// steps s = 0..max_depth attend c_s iff c_s != c_{s-1} (src/ragged_attn.py:
// 338-377 heap, :657-698 parents).  The loads of CH steps are issued together
// (issue) before their scores are formed and folded into the state (fold);
// the walk stops once every lane's walk has stalled (root reached or
// self-loop).  A caller may issue the first chunk before it builds the
// initial state, so those loads overlap its own.
// DBG (walk export): every step's attended node (or -1) is written to dbg[step].
template <typename T, int D, int WALK, int LAYOUT, int CH_ = 8 / (D / 32), bool BATCH = false, bool DBG = false>
struct Walk4 {
    static constexpr int NCH = D / 32;
    static constexpr int CH = CH_;  // default 2 steps at D=128: 64 VGPRs of K/V loads in flight per lane
    const TreeParams& p;
    const int seq;
    const int32_t pb, n;  // parents_base of the sequence, its length
    const int64_t kvb;
    const uint16_t* kb;
    const uint16_t* vb;
    const int32_t tok0;  // the query's own node: the row a step without a key reads
    const uint16_t* qdummy;  // paged: the query's Q row chunk, read by a step without a valid page
    int32_t cur, prev;
    int s0;
    bool val[CH];
    Vec16 kf[CH][NCH], vf[CH][NCH];
    int32_t* dbg;  // DBG only: this query's row of the walk export (written by lane 0 of the group)

    __device__ __forceinline__ Walk4(const TreeParams& p_, int seq_, int32_t start_, int32_t n_, int tok, int kvh,
                                     int j, const uint16_t* qdummy_ = nullptr, int32_t* dbg_ = nullptr)
        : p(p_), seq(seq_), pb(parents_base<BATCH>(p_, seq_, start_)), n(n_), kvb(kv_base(p_, seq_, start_)),
          kb((const uint16_t*)p_.k + (int64_t)kvh * p_.sk_h + 8 * j),
          vb((const uint16_t*)p_.v + (int64_t)kvh * p_.sv_h + 8 * j), tok0(tok), qdummy(qdummy_), cur(tok),
          prev(-1), s0(0), dbg(dbg_) {}

    __device__ __forceinline__ void record(int step, int32_t node) {
        if constexpr (DBG) {
            if (dbg && step <= p.max_depth) dbg[step] = node;
        }
    }

    // Issue the K/V loads of steps s0 .. s0 + CH - 1.  A parents walk asks
    // for each step's next node before that step's K/V rows: loads complete
    // in order, so waiting for the parent leaves the K/V loads in flight, and
    // a chunk costs two round trips rather than one per step plus one.
    // K/V loads are unconditional: a step without a key (past max_depth, a
    // stalled walk) reads the query's own row (packed: in bounds and already
    // attended), or for a paged step without a valid page the query's Q row
    // (in bounds; finite whenever the output can be), and fold gives it score
    // -inf (weight 0).  A guarded load would let the compiler move the fold's
    // conversions behind each load and wait for it there, one round trip per
    // row.
    __device__ __forceinline__ void issue() {
        if constexpr (LAYOUT == KV_PAGED) {
            issue_paged();
            return;
        }
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            bool ok = (s0 + t <= p.max_depth) && (cur != prev);
            int32_t par = 0;
            if constexpr (WALK == WALK_PARENTS) par = p.parents[pb + cur];  // src/ragged_attn.py:692-694
            val[t] = ok;
            record(s0 + t, ok ? cur : -1);
            const int32_t row = ok ? cur : tok0;
            const uint16_t* kr = kb + (kvb + row) * p.sk_t;
            const uint16_t* vr = vb + (kvb + row) * p.sv_t;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                kf[t][i] = ld16(kr + 32 * i);
                vf[t][i] = ld16(vr + 32 * i);
            }
            prev = cur;
            if constexpr (WALK == WALK_PARENTS)
                cur = (par >= 0 && par < n) ? par : cur;
            else
                cur = walk_next<WALK>(p, pb, n, cur);
        }
        // keep the fold's arithmetic below the chunk's loads
        __builtin_amdgcn_sched_barrier(0);
    }

    // Paged K/V (heap walk): the chunk's nodes are arithmetic, so every
    // step's page-table entry is requested before any K/V row and the wait
    // for them leaves no row load behind it (two round trips per chunk).  The
    // entry loads are unconditional too: a logical page past pt_cols reads
    // the row's last entry (or, for an empty table, the Q row) and is
    // discarded.
    __device__ __forceinline__ void issue_paged() {
        int32_t pg[CH], sl[CH], nd[CH];
        bool okn[CH];
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            okn[t] = (s0 + t <= p.max_depth) && (cur != prev);
            nd[t] = cur;
            const int32_t lp = cur / p.page_size;
            sl[t] = cur - lp * p.page_size;
            okn[t] = okn[t] && lp < p.pt_cols;
            const int32_t* ent = p.pt_cols > 0
                                     ? p.page_table + (int64_t)seq * p.pt_cols + min(lp, p.pt_cols - 1)
                                     : (const int32_t*)qdummy;
            pg[t] = *ent;
            prev = cur;
            cur = walk_next<WALK>(p, pb, n, cur);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            const bool ok = okn[t] && pg[t] >= 0 && pg[t] < p.num_pages;
            val[t] = ok;
            record(s0 + t, ok ? nd[t] : -1);
            const uint16_t* kr = ok ? kb + (int64_t)pg[t] * p.sk_page + (int64_t)sl[t] * p.sk_t : qdummy;
            const uint16_t* vr = ok ? vb + (int64_t)pg[t] * p.sv_page + (int64_t)sl[t] * p.sv_t : qdummy;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                kf[t][i] = ld16(kr + 32 * i);
                vf[t][i] = ld16(vr + 32 * i);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // Fold the issued chunk into (m, l, acc) and move to the next chunk.
    __device__ __forceinline__ void fold(const Vec16* qf, float& m, float& l, float* acc) {
        float s[CH];
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            const float d = qk4<T, NCH>(qf, kf[t]) * p.scale_log2;
            s[t] = val[t] ? d : -INFINITY;
        }
        fold_scores<T, NCH, CH>(s, vf, m, l, acc);
        s0 += CH;
    }

    __device__ __forceinline__ bool more() const { return s0 <= p.max_depth && __any(cur != prev); }
};

// Normalise and store one query's output (+ LSE from lane 0 of the group).
template <typename T, int D, bool LSE, bool BATCH = false>
__device__ __forceinline__ void write_out4(const TreeParams& p, int seq, int64_t qrow, int h, int j, float m,
                                           float l, float* acc) {
    constexpr int NCH = D / 32;
    // l == 0 only for a query with no attended key; the reference divides by 1
    // there (src/ragged_attn.py:379-380).
    const float l_safe = (l == 0.f) ? 1.f : l;
    const float inv = __builtin_amdgcn_rcpf(l_safe);
    uint16_t* optr =
        (uint16_t*)p.o + qrow * p.so_t + (BATCH ? (int64_t)seq * p.so_b : 0) + (int64_t)h * p.so_h + 8 * j;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = acc[8 * i + e] * inv;
        st16(optr + 32 * i, pack8<T>(r));
    }
    if constexpr (LSE) {
        if (j == 0)
            p.lse[qrow * p.slse_t + (BATCH ? (int64_t)seq * p.slse_b : 0) + (int64_t)h * p.slse_h] =
                (m + fast_log2(l_safe)) * kLn2;
    }
}

}  // namespace qattn
