// tree_attn.hip -- ancestor-sparse tree-verify attention kernels for gfx950.
//
// Two kernels compute the same function (the ancestor walk + softmax of
// src/ragged_attn.py:262-497):
//
//  * tree_gather_kernel   one row group (D/8 lanes, 16 B per lane) per
//                         (token, q head); the d+1 ancestor rows of a chunk of
//                         steps are gathered from global memory with all loads
//                         issued before the first score is formed.  Handles the
//                         heap walk, the explicit-parent walk and the paged
//                         K/V layout, and merges split-K prefix partial states.
//
//  * tree_stream_kernel   heap trees only (subtree_stream.hip).  Persistent
//                         workgroups walk subtree tiles (a band of BFS levels
//                         under G adjacent roots) of each (sequence, kv head),
//                         staging the tile's K/V rows, the few ancestor rows
//                         above it and its Q rows in LDS while the previous
//                         tile is computed, so each K/V row leaves HBM once per
//                         kv head.  All q heads of a GQA group share the rows.
//                         This file holds its tiling plan (make_subtree_plan).
//
// Scores are kept in the log2 domain (scale * log2(e) folded into one multiply)
// and exponentiated with v_exp_f32.  Dot products use v_dot2_f32_{f16,bf16};
// the D/8-lane reduction uses DPP.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

#include "qattn_common.h"
#include "qattn_device.h"
#include "tree_walk.h"

namespace qattn {

constexpr int kThreads = 256;

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

// The calling thread's walk-export table (qattn_debug_walk), or null.
static thread_local int32_t* g_dbg_walk = nullptr;

// ---------------------------------------------------------------------------
// Gather kernel: 4 lanes per (token, q head), 64 pairs per workgroup with the
// head index fastest, so a workgroup reads 2 tokens' contiguous head rows.
// ---------------------------------------------------------------------------
// DBG: the walk-export instantiation (qattn_debug_walk): every query's walk
// steps are also written to p.dbg_walk.
// TPB: threads per workgroup.  A split merge that would occupy under half
// the CUs (a decode step of a small tree) takes one wave per workgroup
// instead, so four times the CUs share its loads (each CU's vector memory
// path, not latency, bounds such a launch: the EAGLE-3 step's merge of 8
// states over 30 workgroups, 18.62 -> 17.12 us per call).
template <typename T, int D, int WALK, int LAYOUT, bool LSE, bool PSTATE, bool BATCH, bool DBG = false,
          int TPB = kThreads>
__global__ __launch_bounds__(kThreads) void tree_gather_kernel(TreeParams p) {
    constexpr int NCH = D / 32;
    constexpr int SLOTS = TPB / 4;
    const int j = threadIdx.x & 3;
    // Without split states: XCD-contiguous block order.  The dispatcher
    // places block i on XCD i % 8, so XCD x takes the x-th eighth of the
    // logical blocks and neighbouring tokens, whose ancestors coincide, share
    // one L2 (gen1024 -5.3%, cfg2 and cfg3 through this kernel -2% and -5%
    // in A/B runs on one box; with split states the EAGLE-3 step ran 5.6%
    // slower, so that order stays).
    uint32_t lbk = blockIdx.x;
    if constexpr (!PSTATE) {
        const uint32_t nb = gridDim.x, bx = blockIdx.x, per = nb >> 3, rem = nb & 7, x = bx & 7;
        lbk = x * per + min(x, rem) + (bx >> 3);
    }
    const int64_t slot = (int64_t)lbk * SLOTS + (threadIdx.x >> 2);
    int h, tok, seq;
    slot_coords(p, slot, (int64_t)gridDim.x * SLOTS, h, tok, seq);
    if (seq >= p.B) return;
    int32_t start, n;
    if (!seq_bounds<BATCH>(p, seq, start, n)) return;
    if (tok >= n) return;
    const int64_t qrow = (int64_t)start + tok;
    Vec16 qf[NCH];
    load_q4<D, BATCH>(p, seq, qrow, h, j, qf);
    float m = -INFINITY, l = 0.f, acc[8 * NCH];
    // the first chunk of the walk's K/V loads is in flight while the prefix
    // splits are merged (the walk does not depend on them)
    // (a paged step without a valid page reads this query's own Q row)
    const uint16_t* qdummy = (const uint16_t*)p.q + qrow * p.sq_t + (BATCH ? (int64_t)seq * p.sq_b : 0) +
                             (int64_t)h * p.sq_h + 8 * j;
    int32_t* dbg = nullptr;
    if constexpr (DBG) {
        if (j == 0) {
            dbg = p.dbg_walk + (qrow * p.Hq + h) * (p.max_depth + 1);
            for (int i = 0; i <= p.max_depth; ++i) dbg[i] = -1;
        }
    }
    Walk4<T, D, WALK, LAYOUT, 8 / (D / 32), BATCH, DBG> w(p, seq, start, n, tok, h / p.group, j,
                                                          LAYOUT == KV_PAGED ? qdummy : nullptr, dbg);
    w.issue();
    if constexpr (PSTATE) {
        load_partial_state4<T, D>(p, qrow, h, j, m, l, acc);
    } else {
#pragma unroll
        for (int e = 0; e < 8 * NCH; ++e) acc[e] = 0.f;
    }
    w.fold(qf, m, l, acc);
    while (w.more()) {
        w.issue();
        w.fold(qf, m, l, acc);
    }
    write_out4<T, D, LSE, BATCH>(p, seq, qrow, h, j, m, l, acc);
}

// ---------------------------------------------------------------------------
// Ancestor table kernel (debug export of the walk)
// ---------------------------------------------------------------------------
template <int WALK>
__global__ __launch_bounds__(kThreads) void ancestors_kernel(TreeParams p, int32_t* out) {
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int seq = (int)(idx / p.max_seqlen);
    const int tok = (int)(idx % p.max_seqlen);
    if (seq >= p.B) return;
    int32_t start, n;
    if (!seq_bounds(p, seq, start, n)) return;
    if (tok >= n) return;
    int32_t* row = out + ((int64_t)start + tok) * (p.max_depth + 1);
    const int32_t pb = parents_base(p, seq, start);
    int32_t cur = tok, prev = -1;
    for (int s = 0; s <= p.max_depth; ++s) {
        row[s] = (cur != prev) ? cur : -1;
        prev = cur;
        cur = walk_next<WALK>(p, pb, n, cur);
    }
}

// ---------------------------------------------------------------------------
// LSE merge kernel
// ---------------------------------------------------------------------------
struct MergeParams {
    const float* lse_p;
    const float* lse_t;
    const void* o_p;
    const void* o_t;
    void* out;
    int64_t sl_p[3], sl_t[3], so_p[4], so_t[4], so[4];
    int32_t B, H, Nq;
};

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void lse_merge_kernel(MergeParams mp) {
    constexpr int LPR = D / 8;
    constexpr int SLOTS = kThreads / LPR;
    const int lane = threadIdx.x % LPR;
    const int64_t pos = (int64_t)blockIdx.x * SLOTS + threadIdx.x / LPR;
    if (pos >= (int64_t)mp.B * mp.H * mp.Nq) return;
    const int i = (int)(pos % mp.Nq);
    const int h = (int)((pos / mp.Nq) % mp.H);
    const int bb = (int)(pos / ((int64_t)mp.Nq * mp.H));
    const float lp = mp.lse_p[bb * mp.sl_p[0] + h * mp.sl_p[1] + i * mp.sl_p[2]];
    const float lt = mp.lse_t[bb * mp.sl_t[0] + h * mp.sl_t[1] + i * mp.sl_t[2]];
    const float mx = fmaxf(lp, lt);
    const float wp = fast_exp2((lp - mx) * kLog2e);
    const float wt = fast_exp2((lt - mx) * kLog2e);
    const float ws = fmaxf(wp + wt, 1e-8f);
    const Vec16 a = ld16((const uint16_t*)mp.o_p + bb * mp.so_p[0] + h * mp.so_p[1] + i * mp.so_p[2] + lane * 8);
    const Vec16 c = ld16((const uint16_t*)mp.o_t + bb * mp.so_t[0] + h * mp.so_t[1] + i * mp.so_t[2] + lane * 8);
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (wp * elem<T>(a, j) + wt * elem<T>(c, j)) / ws;
    st16((uint16_t*)mp.out + bb * mp.so[0] + h * mp.so[1] + i * mp.so[2] + lane * 8, pack8<T>(r));
}

// ---------------------------------------------------------------------------
// Host side: validation, planning, dispatch
// ---------------------------------------------------------------------------
bool row_aligned(const void* ptr, const int64_t* st, int n_outer) {
    if (((uintptr_t)ptr & 15u) != 0) return false;
    for (int i = 0; i < n_outer; ++i)
        if (st[i] % 8 != 0) return false;
    return st[n_outer] == 1;
}

int check_common(int32_t dtype, int32_t head_dim, int32_t batch, int32_t max_seqlen,
                        int64_t total_tokens, int32_t hq, int32_t hkv, int32_t max_depth) {
    if (dtype != QATTN_DTYPE_F16 && dtype != QATTN_DTYPE_BF16) {
        set_error("dtype %d is not fp16 (0) or bf16 (1)", dtype);
        return QATTN_ERR_DTYPE;
    }
    if (head_dim != 32 && head_dim != 64 && head_dim != 128) {
        set_error("head_dim %d not in {32, 64, 128}", head_dim);
        return QATTN_ERR_HEAD_DIM;
    }
    if (batch < 0 || max_seqlen < 0 || total_tokens < 0 || hq < 1 || hkv < 1 || hq % hkv != 0 ||
        max_depth < 0) {
        set_error("bad sizes: batch=%d max_seqlen=%d total_tokens=%lld hq=%d hkv=%d max_depth=%d", batch,
                  max_seqlen, (long long)total_tokens, hq, hkv, max_depth);
        return QATTN_ERR_ARG;
    }
    if (total_tokens >= (int64_t(1) << 31) || (int64_t)max_seqlen * batch >= (int64_t(1) << 40)) {
        set_error("sizes too large: total_tokens=%lld", (long long)total_tokens);
        return QATTN_ERR_ARG;
    }
    return QATTN_OK;
}

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: %s", what, hipGetErrorString(e));
        return QATTN_ERR_HIP;
    }
    return QATTN_OK;
}

// Subtree tiling plan for a heap tree of n nodes.  Level l of the heap holds
// b^l nodes; a band of levels [lo, hi) is cut into tiles of G roots at level
// lo whose subtrees (down to hi) plus one ancestor row per level above lo fit
// the LDS budget.  Bands are chosen bottom-up, each the tallest that fits a
// single-root subtree.  Returns false when no plan fits the LDS budget.
static bool make_subtree_plan(int b, int64_t n, int max_depth, int rcap, int ncap, SubtreePlan& plan) {
    plan = SubtreePlan{};
    for (int i = 0; i < kMaxBands; ++i) plan.tile_base[i] = INT32_MAX;
    if (n <= 0 || b < 1) return false;
    {
        int64_t st = 0, pw = 1;
        for (int l = 0; l < 64; ++l) {
            plan.lvl_start[l] = (int32_t)std::min<int64_t>(st, INT32_MAX);
            plan.lvl_pow[l] = (uint32_t)std::min<int64_t>(pw, UINT32_MAX);
            if (st < INT32_MAX) st += pw;
            if (pw < UINT32_MAX && b > 1) pw = std::min<int64_t>(pw * b, UINT32_MAX);
        }
    }
    if (b == 1) {
        const int extra = (int)std::min<int64_t>(max_depth, n - 1);
        int h = std::min(rcap - extra, ncap);
        h = std::min(h, 64 - extra);
        if (h < 1) return false;
        h = (int)std::min<int64_t>(h, n);
        plan.nbands = 1;
        plan.chain_h = h;
        plan.tile_base[0] = 0;
        plan.band[0] = 1u << 16;  // lo, hi come from chain_h for b == 1
        const int64_t tiles = (n + h - 1) / h;
        if (tiles >= (int64_t(1) << 30)) return false;
        plan.total_tiles = (int32_t)tiles;
        plan.max_rows = h + extra;
        return true;
    }
    // level starts s[l] and full widths w[l]
    std::vector<int64_t> s, w;
    int64_t sl = 0, wl = 1;
    while (sl < n) {
        s.push_back(sl);
        w.push_back(wl);
        sl += wl;
        if (wl > n) wl = n + 1; else wl *= b;
    }
    const int Lmax = (int)s.size() - 1;
    auto width = [&](int l) -> int64_t { return std::min<int64_t>(w[l], n - s[l]); };
    auto subtree = [&](int h) -> int64_t {  // nodes of one complete root subtree, h levels
        int64_t tot = 0, bj = 1;
        for (int j = 0; j < h; ++j) {
            tot += bj;
            if (tot > rcap) return int64_t(rcap) + 1;
            bj *= b;
        }
        return tot;
    };
    auto extra_rows = [&](int64_t G, int lo) -> int64_t {  // ancestors above G adjacent roots
        int64_t tot = 0, bj = 1;
        const int J = std::min(lo, max_depth);
        for (int j = 1; j <= J; ++j) {
            if (bj <= n) bj *= b;
            const int64_t span = (G - 1 + bj - 1) / bj + 1;
            tot += std::min<int64_t>(span, width(lo - j));
        }
        return tot;
    };
    std::vector<Band> bands;
    int hi = Lmax;
    while (hi >= 0) {
        int best = 0;
        for (int h = 1; h <= hi + 1; ++h) {
            const int lo = hi - h + 1;
            const int nlev = hi - std::max(0, lo - max_depth) + 1;
            if (subtree(h) + extra_rows(1, lo) > rcap || subtree(h) > ncap || nlev > 64) break;
            best = h;
        }
        if (best == 0) return false;
        const int lo = hi - best + 1;
        const int64_t size = subtree(best);
        const int64_t wlo = width(lo);
        int64_t G = 1;
        while (G < wlo && (G + 1) * size + extra_rows(G + 1, lo) <= rcap && (G + 1) * size <= ncap) ++G;
        bands.push_back(Band{lo, hi, (int32_t)G, 0});
        if ((int)bands.size() > kMaxBands) return false;
        hi = lo - 1;
    }
    std::reverse(bands.begin(), bands.end());  // top band first
    int64_t tiles = 0, rows = 0;
    for (size_t i = 0; i < bands.size(); ++i) {
        Band& bd = bands[i];
        bd.tile_base = (int32_t)tiles;
        const int64_t wlo = width(bd.lo);
        tiles += (wlo + bd.G - 1) / bd.G;
        rows = std::max<int64_t>(rows, bd.G * subtree(bd.hi - bd.lo + 1) + extra_rows(bd.G, bd.lo));
        if (bd.hi > 255 || bd.G > 65535) return false;
        plan.tile_base[i] = bd.tile_base;
        plan.band[i] = (uint32_t)bd.lo | ((uint32_t)bd.hi << 8) | ((uint32_t)bd.G << 16);
    }
    if (tiles >= (int64_t(1) << 30)) return false;
    plan.nbands = (int32_t)bands.size();
    plan.total_tiles = (int32_t)tiles;
    plan.max_rows = (int32_t)rows;
    plan.chain_h = 0;
    return rows <= rcap;
}

template <typename T, int D, int WALK, int LAYOUT, bool LSE, bool PSTATE, bool BATCH = false, bool DBG = false>
static int launch_gather(const TreeParams& p, hipStream_t st) {
    constexpr int SLOTS = kThreads / 4;  // 4 lanes per (token, q head)
    const int64_t slots = (int64_t)p.B * p.max_seqlen * p.Hq;
    const int64_t blocks = (slots + SLOTS - 1) / SLOTS;
    if (blocks >= (int64_t(1) << 31)) {
        set_error("grid too large (%lld blocks)", (long long)blocks);
        return QATTN_ERR_ARG;
    }
    if constexpr (PSTATE && LAYOUT == KV_PACKED) {
        if (blocks < 128) {  // (cfg4's merge, 170 workgroups, timed within noise either way)
            constexpr int S1 = 64 / 4;
            hipLaunchKernelGGL((tree_gather_kernel<T, D, WALK, LAYOUT, LSE, PSTATE, BATCH, DBG, 64>),
                               dim3((unsigned)((slots + S1 - 1) / S1)), dim3(64), 0, st, p);
            return launch_status("tree_gather_kernel");
        }
    }
    hipLaunchKernelGGL((tree_gather_kernel<T, D, WALK, LAYOUT, LSE, PSTATE, BATCH, DBG>), dim3((unsigned)blocks),
                       dim3(kThreads), 0, st, p);
    return launch_status("tree_gather_kernel");
}

template <typename T, int D, int WALK, bool BATCH>
static int gather_packed(const TreeParams& p, bool lse, bool pstate, hipStream_t st) {
    if (pstate) {
        return lse ? launch_gather<T, D, WALK, KV_PACKED, true, true, BATCH>(p, st)
                   : launch_gather<T, D, WALK, KV_PACKED, false, true, BATCH>(p, st);
    }
    return lse ? launch_gather<T, D, WALK, KV_PACKED, true, false, BATCH>(p, st)
               : launch_gather<T, D, WALK, KV_PACKED, false, false, BATCH>(p, st);
}

// Walk export (qattn_debug_walk): the walk-export instantiation of the gather
// kernel that serves the same call (dtype, LSE, walk, layout, prefix state).
template <typename T, int D, bool LSE>
static int gather_dbg(const TreeParams& p, int walk, int layout, bool pstate, hipStream_t st) {
    if (layout == KV_PAGED) return launch_gather<T, D, WALK_HEAP, KV_PAGED, LSE, false, false, true>(p, st);
    if (walk == WALK_HEAP)
        return pstate ? launch_gather<T, D, WALK_HEAP, KV_PACKED, LSE, true, false, true>(p, st)
                      : launch_gather<T, D, WALK_HEAP, KV_PACKED, LSE, false, false, true>(p, st);
    return pstate ? launch_gather<T, D, WALK_PARENTS, KV_PACKED, LSE, true, false, true>(p, st)
                  : launch_gather<T, D, WALK_PARENTS, KV_PACKED, LSE, false, false, true>(p, st);
}

template <typename T, int D>
static int dispatch_tree(const TreeParams& p, int walk, int layout, bool lse, bool pstate, int algo,
                         hipStream_t st) {
    const bool paged = layout == KV_PAGED;
    if (walk == WALK_HEAP && (!paged || !pstate) && algo != QATTN_ALGO_GATHER) {
        SubtreePlan plan;
        int rcap = 0, qcap = 0;
        stream_tile_caps(D, &rcap, &qcap);
        // (paged: the page table is copied to LDS, so it has a size limit, and
        // one 32-bit offset addresses K and V: equal strides below 2^31)
        const bool paged_ok = !paged || ((int64_t)p.B * p.pt_cols <= stream_max_page_entries() &&
                                         p.sk_page == p.sv_page && p.sk_t == p.sv_t && p.sk_h == p.sv_h &&
                                         p.sk_page >= 0 && p.sk_page < (int64_t(1) << 31) && p.sk_t >= 0 &&
                                         p.sk_t < (int64_t(1) << 31) && p.page_size <= 4096 &&
                                         (p.max_seqlen - 1) / p.page_size < (1 << 19));
        const bool ok = p.B <= stream_max_batch() && paged_ok &&
                        make_subtree_plan(p.bdiv.d, p.max_seqlen, p.max_depth, rcap, qcap / p.group, plan);
        const int64_t wgs = ok ? (int64_t)p.B * p.Hkv * plan.total_tiles : 0;
        // The subtree kernel needs enough tiles to fill 256 CUs; a merged
        // prefix state makes each query heavier, so it only pays off there
        // when tiles are plentiful.
        const bool use = ok && (algo == QATTN_ALGO_SUBTREE || wgs >= (pstate ? 2048 : 512));
        if (algo == QATTN_ALGO_SUBTREE && !ok) {
            if (!paged_ok)
                set_error("paged subtree kernel: page-table entries %lld (at most %d), page size %d (at most "
                          "4096), or K/V cache strides that differ or reach 2^31",
                          (long long)p.B * p.pt_cols, stream_max_page_entries(), p.page_size);
            else
                set_error("no subtree plan fits (b=%d, max_seqlen=%d, max_depth=%d, batch=%d)", p.bdiv.d,
                          p.max_seqlen, p.max_depth, p.B);
            return QATTN_ERR_ARG;
        }
        if (use) return launch_stream(p, plan, T::kCode, D, pstate, paged, st);
    } else if (algo == QATTN_ALGO_SUBTREE) {
        set_error("the subtree kernel supports the heap walk on packed or paged K/V only");
        return QATTN_ERR_ARG;
    }
    if (p.dbg_walk) {
        // walk export: calls over packed cu_seqlens, either dtype, with or without LSE
        if (!p.cu) {
            set_error("the walk export runs calls over packed cu_seqlens");
            return QATTN_ERR_ARG;
        }
        return lse ? gather_dbg<T, D, true>(p, walk, layout, pstate, st)
                   : gather_dbg<T, D, false>(p, walk, layout, pstate, st);
    }
    if (layout == KV_PACKED) {
        // (a null cu is a uniform batch: its addressing is compiled separately)
        if (!p.cu) {
            return walk == WALK_HEAP ? gather_packed<T, D, WALK_HEAP, true>(p, lse, pstate, st)
                                     : gather_packed<T, D, WALK_PARENTS, true>(p, lse, pstate, st);
        }
        return walk == WALK_HEAP ? gather_packed<T, D, WALK_HEAP, false>(p, lse, pstate, st)
                                 : gather_packed<T, D, WALK_PARENTS, false>(p, lse, pstate, st);
    }
    return lse ? launch_gather<T, D, WALK_HEAP, KV_PAGED, true, false>(p, st)
               : launch_gather<T, D, WALK_HEAP, KV_PAGED, false, false>(p, st);
}

int run_tree(const TreeParams& p, int dtype, int head_dim, int walk, int layout, bool pstate, int algo,
             hipStream_t st) {
    const bool lse = p.lse != nullptr;
    if (dtype == QATTN_DTYPE_F16) {
        switch (head_dim) {
            case 32: return dispatch_tree<F16, 32>(p, walk, layout, lse, pstate, algo, st);
            case 64: return dispatch_tree<F16, 64>(p, walk, layout, lse, pstate, algo, st);
            default: return dispatch_tree<F16, 128>(p, walk, layout, lse, pstate, algo, st);
        }
    }
    switch (head_dim) {
        case 32: return dispatch_tree<BF16, 32>(p, walk, layout, lse, pstate, algo, st);
        case 64: return dispatch_tree<BF16, 64>(p, walk, layout, lse, pstate, algo, st);
        default: return dispatch_tree<BF16, 128>(p, walk, layout, lse, pstate, algo, st);
    }
}

// Fill the fields shared by the tree entry points.  Returns an error code.
int fill_tree_params(TreeParams& p, const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                     const void* v, const int64_t* vs, void* o, const int64_t* os, float* lse,
                     const int64_t* lss, const int32_t* cu, int32_t batch, int32_t max_seqlen,
                     int64_t total_tokens, int32_t hq, int32_t hkv, int32_t b, int32_t max_depth, float scale,
                     bool uniform) {
    p = TreeParams{};
    if (!q || !qs || !k || !ks || !v || !vs || !o || !os || (!cu && !uniform) || (lse && !lss)) {
        set_error("null pointer argument");
        return QATTN_ERR_ARG;
    }
    if (b < 1) {
        set_error("branching_factor %d < 1", b);
        return QATTN_ERR_ARG;
    }
    if (!row_aligned(q, qs, 2) || !row_aligned(o, os, 2)) {
        set_error("q/o rows must be 16-byte aligned with stride_dim 1");
        return QATTN_ERR_LAYOUT;
    }
    if (!(scale == scale)) {
        set_error("scale is NaN");
        return QATTN_ERR_ARG;
    }
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.lse = lse;
    p.cu = cu;
    p.sq_t = qs[0];
    p.sq_h = qs[1];
    p.sk_t = ks[0];
    p.sk_h = ks[1];
    p.sv_t = vs[0];
    p.sv_h = vs[1];
    p.so_t = os[0];
    p.so_h = os[1];
    if (lse) {
        p.slse_t = lss[0];
        p.slse_h = lss[1];
    }
    p.total_tokens = total_tokens;
    p.kv_rows = total_tokens;
    p.B = batch;
    p.Hq = hq;
    p.Hkv = hkv;
    p.group = hq / hkv;
    p.max_seqlen = max_seqlen;
    p.max_depth = max_depth;
    p.bdiv = make_divider(b);
    p.hqdiv = make_divider(hq);
    p.msdiv = make_divider(max_seqlen > 0 ? max_seqlen : 1);
    p.scale_log2 = scale * kLog2e;
    p.dbg_walk = g_dbg_walk;
    return QATTN_OK;
}

}  // namespace qattn

using namespace qattn;

extern "C" {

const char* qattn_version(void) { return "qattention_amd 0.1.0 (gfx950)"; }

const char* qattn_last_error(void) { return g_err; }

int qattn_debug_walk(int32_t* out) {
    g_dbg_walk = out;
    return QATTN_OK;
}

int qattn_tree_fwd(const void* q, const int64_t q_stride[3], const void* k, const int64_t k_stride[3],
                   const void* v, const int64_t v_stride[3], void* o, const int64_t o_stride[3], float* lse,
                   const int64_t lse_stride[2], const int32_t* cu_seqlens, int32_t batch, int32_t max_seqlen,
                   int64_t total_tokens, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                   int32_t branching_factor, int32_t max_depth, float scale, int32_t dtype, int32_t algo,
                   void* stream) {
    clear_error();
    int rc = check_common(dtype, head_dim, batch, max_seqlen, total_tokens, num_q_heads, num_kv_heads, max_depth);
    if (rc) return rc;
    if (algo < QATTN_ALGO_AUTO || algo > QATTN_ALGO_SUBTREE) {
        set_error("unknown algo %d", algo);
        return QATTN_ERR_ARG;
    }
    if (batch == 0 || max_seqlen == 0 || total_tokens == 0) return QATTN_OK;  // nothing to compute
    TreeParams p;
    rc = fill_tree_params(p, q, q_stride, k, k_stride, v, v_stride, o, o_stride, lse, lse_stride, cu_seqlens,
                          batch, max_seqlen, total_tokens, num_q_heads, num_kv_heads, branching_factor, max_depth,
                          scale);
    if (rc) return rc;
    if (!row_aligned(k, k_stride, 2) || !row_aligned(v, v_stride, 2)) {
        set_error("k/v rows must be 16-byte aligned with stride_dim 1");
        return QATTN_ERR_LAYOUT;
    }
    return run_tree(p, dtype, head_dim, WALK_HEAP, KV_PACKED, false, algo, (hipStream_t)stream);
}

int qattn_tree_parents_fwd(const void* q, const int64_t q_stride[3], const void* k, const int64_t k_stride[3],
                           const void* v, const int64_t v_stride[3], void* o, const int64_t o_stride[3],
                           float* lse, const int64_t lse_stride[2], const int32_t* cu_seqlens,
                           const int32_t* parents, int32_t batch, int32_t max_seqlen, int64_t total_tokens,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t max_depth,
                           float scale, int32_t dtype, void* stream) {
    clear_error();
    int rc = check_common(dtype, head_dim, batch, max_seqlen, total_tokens, num_q_heads, num_kv_heads, max_depth);
    if (rc) return rc;
    if (batch == 0 || max_seqlen == 0 || total_tokens == 0) return QATTN_OK;  // nothing to compute
    if (!parents) {
        set_error("parents is null");
        return QATTN_ERR_ARG;
    }
    TreeParams p;
    rc = fill_tree_params(p, q, q_stride, k, k_stride, v, v_stride, o, o_stride, lse, lse_stride, cu_seqlens,
                          batch, max_seqlen, total_tokens, num_q_heads, num_kv_heads, 1, max_depth, scale);
    if (rc) return rc;
    if (!row_aligned(k, k_stride, 2) || !row_aligned(v, v_stride, 2)) {
        set_error("k/v rows must be 16-byte aligned with stride_dim 1");
        return QATTN_ERR_LAYOUT;
    }
    p.parents = parents;
    return run_tree(p, dtype, head_dim, WALK_PARENTS, KV_PACKED, false, QATTN_ALGO_GATHER, (hipStream_t)stream);
}

int qattn_tree_paged_fwd(const void* q, const int64_t q_stride[3], const void* k_cache, const int64_t k_stride[4],
                         const void* v_cache, const int64_t v_stride[4], void* o, const int64_t o_stride[3],
                         float* lse, const int64_t lse_stride[2], const int32_t* cu_seqlens,
                         const int32_t* page_table, int32_t pt_cols, int32_t num_pages, int32_t page_size,
                         int32_t batch, int32_t max_seqlen, int64_t total_tokens, int32_t num_q_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t branching_factor, int32_t max_depth,
                         float scale, int32_t dtype, int32_t algo, void* stream) {
    clear_error();
    int rc = check_common(dtype, head_dim, batch, max_seqlen, total_tokens, num_q_heads, num_kv_heads, max_depth);
    if (rc) return rc;
    if (algo < QATTN_ALGO_AUTO || algo > QATTN_ALGO_SUBTREE) {
        set_error("unknown algo %d", algo);
        return QATTN_ERR_ARG;
    }
    if (batch == 0 || max_seqlen == 0 || total_tokens == 0) return QATTN_OK;  // nothing to compute
    if (!page_table || !k_stride || !v_stride || page_size < 1 || pt_cols < 0 || num_pages < 0) {
        set_error("bad paged arguments: page_size=%d pt_cols=%d num_pages=%d", page_size, pt_cols, num_pages);
        return QATTN_ERR_ARG;
    }
    // The walk's K/V access is page * stride_page + slot * stride_slot + head * stride_head.
    const int64_t ks3[3] = {k_stride[1], k_stride[2], k_stride[3]};
    const int64_t vs3[3] = {v_stride[1], v_stride[2], v_stride[3]};
    TreeParams p;
    rc = fill_tree_params(p, q, q_stride, k_cache, ks3, v_cache, vs3, o, o_stride, lse, lse_stride, cu_seqlens,
                          batch, max_seqlen, total_tokens, num_q_heads, num_kv_heads, branching_factor, max_depth,
                          scale);
    if (rc) return rc;
    if (!row_aligned(k_cache, ks3, 2) || !row_aligned(v_cache, vs3, 2) || k_stride[0] % 8 || v_stride[0] % 8) {
        set_error("k/v cache rows must be 16-byte aligned with stride_dim 1");
        return QATTN_ERR_LAYOUT;
    }
    p.page_table = page_table;
    p.pt_cols = pt_cols;
    p.num_pages = num_pages;
    p.page_size = page_size;
    p.pdiv = make_divider(page_size);
    p.sk_page = k_stride[0];
    p.sv_page = v_stride[0];
    return run_tree(p, dtype, head_dim, WALK_HEAP, KV_PAGED, false, algo, (hipStream_t)stream);
}

int qattn_ancestors(const int32_t* cu_seqlens, const int32_t* parents, int32_t batch, int32_t max_seqlen,
                    int64_t total_tokens, int32_t branching_factor, int32_t max_depth, int32_t* out,
                    void* stream) {
    clear_error();
    if (!cu_seqlens || !out || batch < 0 || max_seqlen < 0 || total_tokens < 0 || max_depth < 0 ||
        (!parents && branching_factor < 1) || total_tokens >= (int64_t(1) << 31)) {
        set_error("bad arguments to qattn_ancestors");
        return QATTN_ERR_ARG;
    }
    if (batch == 0 || max_seqlen == 0 || total_tokens == 0) return QATTN_OK;
    TreeParams p{};
    p.cu = cu_seqlens;
    p.parents = parents;
    p.B = batch;
    p.max_seqlen = max_seqlen;
    p.total_tokens = total_tokens;
    p.max_depth = max_depth;
    p.bdiv = make_divider(parents ? 1 : branching_factor);
    const int64_t n = (int64_t)batch * max_seqlen;
    const int64_t blocks = (n + kThreads - 1) / kThreads;
    if (parents)
        hipLaunchKernelGGL(ancestors_kernel<WALK_PARENTS>, dim3((unsigned)blocks), dim3(kThreads), 0,
                           (hipStream_t)stream, p, out);
    else
        hipLaunchKernelGGL(ancestors_kernel<WALK_HEAP>, dim3((unsigned)blocks), dim3(kThreads), 0,
                           (hipStream_t)stream, p, out);
    return launch_status("ancestors_kernel");
}

int qattn_lse_merge(const float* lse_pre, const int64_t lse_pre_stride[3], const float* lse_tree,
                    const int64_t lse_tree_stride[3], const void* o_pre, const int64_t o_pre_stride[4],
                    const void* o_tree, const int64_t o_tree_stride[4], void* out, const int64_t out_stride[4],
                    int32_t B, int32_t H, int32_t Nq, int32_t head_dim, int32_t dtype, void* stream) {
    clear_error();
    if (!lse_pre || !lse_tree || !o_pre || !o_tree || !out || !lse_pre_stride || !lse_tree_stride ||
        !o_pre_stride || !o_tree_stride || !out_stride || B < 0 || H < 0 || Nq < 0) {
        set_error("bad arguments to qattn_lse_merge");
        return QATTN_ERR_ARG;
    }
    if (dtype != QATTN_DTYPE_F16 && dtype != QATTN_DTYPE_BF16) {
        set_error("dtype %d is not fp16 (0) or bf16 (1)", dtype);
        return QATTN_ERR_DTYPE;
    }
    if (head_dim != 32 && head_dim != 64 && head_dim != 128) {
        set_error("head_dim %d not in {32, 64, 128}", head_dim);
        return QATTN_ERR_HEAD_DIM;
    }
    if (!row_aligned(o_pre, o_pre_stride, 3) || !row_aligned(o_tree, o_tree_stride, 3) ||
        !row_aligned(out, out_stride, 3)) {
        set_error("merge operands must have stride_dim 1 and 16-byte aligned rows");
        return QATTN_ERR_LAYOUT;
    }
    const int64_t npos = (int64_t)B * H * Nq;
    if (npos == 0) return QATTN_OK;
    MergeParams mp{};
    mp.lse_p = lse_pre;
    mp.lse_t = lse_tree;
    mp.o_p = o_pre;
    mp.o_t = o_tree;
    mp.out = out;
    for (int i = 0; i < 3; ++i) {
        mp.sl_p[i] = lse_pre_stride[i];
        mp.sl_t[i] = lse_tree_stride[i];
    }
    for (int i = 0; i < 4; ++i) {
        mp.so_p[i] = o_pre_stride[i];
        mp.so_t[i] = o_tree_stride[i];
        mp.so[i] = out_stride[i];
    }
    mp.B = B;
    mp.H = H;
    mp.Nq = Nq;
    const int slots = kThreads / (head_dim / 8);
    const int64_t blocks = (npos + slots - 1) / slots;
    if (blocks >= (int64_t(1) << 31)) {
        set_error("grid too large");
        return QATTN_ERR_ARG;
    }
    hipStream_t st = (hipStream_t)stream;
#define QATTN_MERGE(T, D) \
    hipLaunchKernelGGL((lse_merge_kernel<T, D>), dim3((unsigned)blocks), dim3(kThreads), 0, st, mp)
    if (dtype == QATTN_DTYPE_F16) {
        if (head_dim == 32) QATTN_MERGE(F16, 32);
        else if (head_dim == 64) QATTN_MERGE(F16, 64);
        else QATTN_MERGE(F16, 128);
    } else {
        if (head_dim == 32) QATTN_MERGE(BF16, 32);
        else if (head_dim == 64) QATTN_MERGE(BF16, 64);
        else QATTN_MERGE(BF16, 128);
    }
#undef QATTN_MERGE
    return launch_status("lse_merge_kernel");
}

}  // extern "C"
