// subtree_stream.hip -- persistent, software-pipelined subtree kernel for the
// heap ancestor walk (src/ragged_attn.py:262-387 over complete b-ary heaps).
//
// Tiling: the heap parent (i-1)/b makes the ancestors of a subtree a union of
// contiguous BFS level ranges, so the host cuts each tree into tiles (a band
// of levels under G adjacent roots, plus one ancestor row per level above the
// band; make_subtree_plan in tree_attn.hip).  Every K/V row of a tile is read
// from HBM once per kv head, and every ancestor read is an LDS read.
//
// Pipeline: each workgroup is persistent.  Right after tile i is written to
// LDS, the workgroup issues the global loads of tile i+1 (its K and V rows and
// the Q rows of its queries) into registers and then computes tile i from
// LDS, so HBM sees a steady stream of requests.  The workgroups of a group
// share one tile index (so a workgroup keeps its level table and load
// addresses) and take that index's (sequence, kv head) items from the group's
// atomic counter, one item ahead; without a counter slot (see sched_counters)
// workgroup j of a group takes items j, j + n, j + 2n, ... of its n-workgroup
// group instead.
//
// Compute, on the matrix cores: a tile holds at most 48 (D = 128) or 64 K/V
// rows and as many queries, so attention over the tile is three small dense
// products per 16-query block (one wave):
//   S^T = K Q^T                 v_mfma_f32_16x16x32, keys x queries
//   mask: a query attends exactly the rows of its ancestor walk (a 64-bit row
//         mask per query), everything else is -inf
//   P = exp2(S c - m c), one softmax per query column (max and sum over the
//       4 lanes holding the column)
//   O^T = V^T P^T               P split into hi + lo halves of T, so the
//                               products keep fp32 accuracy in P
// V stays row-major in LDS like K: the V^T operand of the PV product is read
// with gfx950's transposing LDS load (ds_read_b64_tr_b16), two per MFMA, in
// the key order in which the S^T output registers form the P^T operand.
#include <algorithm>
#include <mutex>

#include "qattn_common.h"
#include "qattn_device.h"
#include "tree_walk.h"

namespace qattn {

constexpr int kStThreads = 256;
constexpr int kCuCache = 256;  // cu_seqlens entries cached in LDS
constexpr int kPtCache = 2048; // paged K/V: page-table entries cached in LDS (B * pt_cols)
// s_waitcnt immediate (gfx9 encoding): vmcnt 0, expcnt and lgkmcnt unconstrained
constexpr int kWaitVmcnt0 = (7 << 4) | (15 << 8);

// Per-query facts of a tile that depend only on the tile's shape (tile index
// and sequence length), kept in LDS while a workgroup stays on one tile: the
// rows the query attends (bit r = K/V row r), its node and q-head offset.
struct alignas(16) QueryEntry {
    uint32_t mask_lo, mask_hi;
    int32_t node, hoff;
};

template <int D>
struct StreamGeom {
    static constexpr int CPR = D / 8;                 // 16-byte chunks per row
    static constexpr int RPP = kStThreads / CPR;      // rows per staging pass
    static constexpr int PASSES = D == 128 ? 3 : (D == 64 ? 2 : 1);
    static constexpr int KV_ROWS = PASSES * RPP;      // K/V rows per tile (48 or 64)
    static constexpr int Q_ROWS = KV_ROWS;            // queries per tile
    static constexpr int PITCH = D + 16;              // K, V and Q row pitch (elements)
    static constexpr int V_ROWS = KV_ROWS;            // V rows the PV product reads
    static constexpr int KT = KV_ROWS / 16;           // 16-key tiles of S^T
    static constexpr int NC = D / 32;                 // 32-element k-chunks of Q K^T
    static constexpr int ND = D / 16;                 // 16-row d-tiles of O^T
    static constexpr size_t LDS_BYTES = ((size_t)(KV_ROWS + Q_ROWS + V_ROWS) * PITCH) * 2 +
                                        (size_t)2 * Q_ROWS * sizeof(QueryEntry) + kCuCache * 4 + 16 + 128 * 4;
    // walk export only: the staged row maps (node of each K/V row, token and
    // head offset of each Q row)
    static constexpr size_t DBG_BYTES = (size_t)(KV_ROWS + Q_ROWS) * 4;
    // paged K/V only: one flag per K/V row (its page exists) for two tiles,
    // then the page table (B * pt_cols entries)
    static constexpr size_t ROWOK_BYTES = (size_t)2 * KV_ROWS * 4;
};

// Per-tile state.  Scalars are wave-uniform; first/cnt/off/qb are per lane,
// lane i describing BFS level lam_min + i (its first node, node count, LDS row
// offset = row - node, and first Q row).
struct TileMeta {
    int32_t valid, tile, seq, kvh, start, n, lo, lam_min, nlev, rows, nq;
    int64_t kvb;
    int32_t first, cnt, off, qb;
};

// Rows of this thread's loads of a tile (chunk tid % CPR of each): K/V pass ps
// stages LDS row ps * RPP + tid / CPR, which is K/V row kvrow[ps] past the
// tile's kv base; Q pass ps stages Q row ps * RPP + tid / CPR, which is token
// qrow[ps] >> 8 past the tile's start at q head qrow[ps] & 255 past the kv
// head's first.  They depend only on the level table, so a workgroup that
// stays on one tile computes them once; 32-bit rows keep them in few
// registers (the 64-bit element offsets are formed at issue).
template <int D>
struct RowMap {
    int32_t kvrow[StreamGeom<D>::PASSES], qrow[StreamGeom<D>::PASSES];
};

template <int D>
struct Stage {
    Vec16 k[StreamGeom<D>::PASSES], v[StreamGeom<D>::PASSES], q[StreamGeom<D>::PASSES];
};

int stream_max_batch() { return kCuCache - 1; }
int stream_max_page_entries() { return kPtCache; }

void stream_tile_caps(int head_dim, int* kv_rows, int* q_rows) {
    const int rows = head_dim == 128 ? StreamGeom<128>::KV_ROWS
                                     : (head_dim == 64 ? StreamGeom<64>::KV_ROWS : StreamGeom<32>::KV_ROWS);
    *kv_rows = rows;
    *q_rows = rows;
}

// Sequence of tile index w = (seq * Hkv + kvh) * tiles + tile.
__device__ __forceinline__ int tile_seq(const StreamArgs& sa, int w) {
    return divide(divide(w, sa.tiles_div), sa.hkv_div);
}

// Inclusive prefix sum over the 64 lanes of a wave: row_shr steps within
// each 16-lane row (lanes without a source add 0), then the row totals.
__device__ __forceinline__ int wave_incl_sum(int x) {
    int v = x;
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);  // row_shr:8
    const int lane = threadIdx.x & 63;
    const int t0 = __builtin_amdgcn_readlane(v, 15), t1 = __builtin_amdgcn_readlane(v, 31),
              t2 = __builtin_amdgcn_readlane(v, 47);
    return v + (lane >= 16 ? t0 : 0) + (lane >= 32 ? t1 : 0) + (lane >= 48 ? t2 : 0);
}

// Lane i's value of x on every lane that asks for lane idx (0..63).
__device__ __forceinline__ int lane_get(int x, int idx) { return __builtin_amdgcn_ds_bpermute(idx << 2, x); }

// Which tile w is, and its level table (src/ragged_attn.py:376-377 walk:
// the ancestors of roots r0..r1-1 at level lo are, per level, one contiguous
// node range), for a sequence spanning tokens [s, e) (cu_seqlens[seq],
// cu_seqlens[seq + 1], wave-uniform).  Returns true when the level table was
// (re)computed, false when it was taken from prev (same tile index and
// sequence length).  bpk / tbase: the tile's band (lo | hi << 8 | G << 16)
// and the band's first tile; lvl_st / lvl_pw: lane l holds plan.lvl_start[l]
// / plan.lvl_pow[l]; when HAVE_LVL is false they are read here from lvl_lds,
// the workgroup's LDS copy (a global load in this rarely taken path would
// make the compiler wait for every load in flight, the next tile's included,
// before the compute).
//
// Every lane works out its own level from the plan's level tables with a few
// independent operations (the descendants j levels below the root range
// [r0, r1) span r0 b^j + start(j) .. r1 b^j + start(j) - 1; the ancestors k
// levels above it are (r0 - start(k)) / b^k .. (r1 - 1 - start(k)) / b^k),
// and the row and query bases are wave prefix sums: the chain from the first
// tile's sequence bounds to its first loads stays short.
template <int D, bool HAVE_LVL>
__device__ __forceinline__ bool tile_setup_se(const TreeParams& p, const SubtreePlan& plan, const StreamArgs& sa,
                                              int w, int32_t s, int32_t e, const TileMeta& prev, TileMeta& t,
                                              uint32_t bpk, int tbase, int32_t lvl_st, uint32_t lvl_pw,
                                              const int32_t* lvl_lds) {
    const int lane = threadIdx.x & 63;
    t.valid = 0;
    t.rows = t.nq = 0;
    t.nlev = 0;
    t.lo = 0;
    t.lam_min = 0;
    t.start = t.n = 0;
    t.kvb = 0;
    t.first = t.cnt = t.off = t.qb = 0;
    // w = (seq * Hkv + kvh) * tiles + tile: with a grid that is a multiple of
    // the tile count, a workgroup keeps one tile index for its whole life.
    const int pair = divide(w, sa.tiles_div);
    const int tile = w - pair * plan.total_tiles;
    const int seq = divide(pair, sa.hkv_div);
    t.tile = tile;
    t.seq = seq;
    t.kvh = pair - seq * p.Hkv;
    if (seq >= p.B) return true;
    if (s < 0 || e < s || (int64_t)e > p.total_tokens) return true;
    int32_t n = e - s;
    if (n > p.max_seqlen) n = p.max_seqlen;
    if (n <= 0) return true;
    if (prev.valid && prev.tile == tile && prev.n == n) {
        t = prev;
        t.seq = seq;
        t.kvh = pair - seq * p.Hkv;
        t.start = s;
        t.kvb = kv_base(p, seq, s);
        return false;
    }
    if constexpr (!HAVE_LVL) {
        lvl_st = lvl_lds[lane];
        lvl_pw = (uint32_t)lvl_lds[64 + lane];
    }
    const int b = p.bdiv.d;
    int lo = (int)(bpk & 255u), hi = (int)((bpk >> 8) & 255u);
    const int G = (int)(bpk >> 16);
    int64_t r0, r1;  // root range [r0, r1) at level lo
    if (b == 1) {
        lo = (tile - tbase) * plan.chain_h;
        hi = lo + plan.chain_h - 1;
        r0 = lo;
        r1 = lo + 1;
    } else {
        const int64_t s_lo = __builtin_amdgcn_readlane(lvl_st, lo);
        const int64_t w_lo = (uint32_t)__builtin_amdgcn_readlane((int)lvl_pw, lo);
        const int64_t i0 = (int64_t)(tile - tbase) * G;
        r0 = s_lo + i0;
        r1 = s_lo + ((i0 + G < w_lo) ? i0 + G : w_lo);
    }
    if (r0 >= n) return true;
    if (r1 > n) r1 = n;

    const int lam_min = (lo - p.max_depth > 0) ? lo - p.max_depth : 0;
    const int nlev = hi - lam_min + 1;  // <= 64, guaranteed by the host plan
    const int lam = lam_min + lane;
    // level offset from the root level: j >= 0 below, -j above
    const int j = lam - lo;
    const int aj = j >= 0 ? j : -j;
    const int32_t st_j = lane_get(lvl_st, aj < 63 ? aj : 63);
    const uint32_t pw_j = (uint32_t)lane_get((int)lvl_pw, aj < 63 ? aj : 63);
    int64_t f, la;
    if (j >= 0) {
        f = (int64_t)((uint64_t)r0 * pw_j) + st_j;
        la = (int64_t)((uint64_t)r1 * pw_j) + st_j - 1;
    } else {
        f = (uint32_t)(r0 - st_j) / pw_j;
        la = (uint32_t)(r1 - 1 - st_j) / pw_j;
    }
    if (la > n - 1) la = n - 1;
    int first = 0, cnt = 0;
    if (lane < nlev && f <= la) {
        first = (int)f;
        cnt = (int)(la - f + 1);
    }
    // exclusive prefix sums over levels: K/V LDS row base, Q LDS row base
    const int qc = (lane < nlev && j >= 0) ? cnt * p.group : 0;
    const int cend = wave_incl_sum(cnt), qend = wave_incl_sum(qc);
    const int rows = __builtin_amdgcn_readlane(cend, nlev - 1);
    const int nq = __builtin_amdgcn_readlane(qend, nlev - 1);
    if (rows > StreamGeom<D>::KV_ROWS || nq > StreamGeom<D>::Q_ROWS) return true;  // not for a host-built plan
    t.start = s;
    t.n = n;
    t.lo = lo;
    t.lam_min = lam_min;
    t.nlev = nlev;
    t.rows = rows;
    t.nq = nq;
    t.kvb = kv_base(p, seq, s);
    t.first = first;
    t.cnt = cnt;
    t.off = cend - cnt - first;
    t.qb = qend - qc;
    t.valid = 1;
    return true;
}

// tile_setup_se with the sequence bounds from the workgroup's LDS copy of
// cu_seqlens (the host launches this kernel only for B < kCuCache): a global
// load here would make the wait for it also wait for every O store still in
// flight.  readfirstlane: the offsets are wave-uniform, so every tile scalar
// derived from them stays in SGPRs and every branch on them is a scalar branch.
template <int D>
__device__ __forceinline__ bool tile_setup(const TreeParams& p, const SubtreePlan& plan, const StreamArgs& sa,
                                           const int32_t __attribute__((address_space(3)))* cu_lds, int w,
                                           const TileMeta& prev, TileMeta& t, int32_t band_tb, uint32_t band_pk,
                                           const int32_t* lvl_lds) {
    int seq = tile_seq(sa, w);
    seq = seq < p.B ? seq : p.B;  // tile_setup_se rejects seq >= B
    const int32_t s = __builtin_amdgcn_readfirstlane(cu_lds[seq]);
    const int32_t e = __builtin_amdgcn_readfirstlane(cu_lds[seq < p.B ? seq + 1 : seq]);
    // the tile's band: bands cover ascending tile ranges from tile 0
    const int tile = w - divide(w, sa.tiles_div) * plan.total_tiles;
    const int bi = (int)__builtin_popcountll(__ballot(tile >= band_tb)) - 1;
    const uint32_t bpk = (uint32_t)__builtin_amdgcn_readlane((int)band_pk, bi);
    const int tbase = __builtin_amdgcn_readlane(band_tb, bi);
    return tile_setup_se<D, false>(p, plan, sa, w, s, e, prev, t, bpk, tbase, 0, 0u, lvl_lds);
}

// The load rows of a tile (RowMap) from its level table.  Lane x of each
// wave works out K/V row x and Q row x of the tile (one pass over the levels
// with wave-uniform values: row x lies in the last level whose base is <= x),
// then every thread takes the rows it stages from those lanes.
// PAGED: kvrow holds the row's logical page << kSlotBits | its slot in the
// page instead of its node (the host keeps page_size <= 2^kSlotBits and the
// logical pages below 2^(31 - kSlotBits)), so the tile loop needs neither
// the page size nor its divider.
constexpr int kSlotBits = 12;
template <int D, bool PAGED = false>
__device__ __forceinline__ void tile_rowmap(const TreeParams& p, const Divider& gdiv, const TileMeta& t,
                                            RowMap<D>& rm) {
    using Geo = StreamGeom<D>;
    static_assert(Geo::KV_ROWS <= 64 && Geo::Q_ROWS <= 64, "one row per lane");
    // (nlev <= 64, so z is 0: it keeps the lane and row terms below inside
    // this rarely taken path instead of live across the whole tile loop)
    const int z = t.nlev >> 7;
    const int x = (threadIdx.x + z) & 63;
    int koff = rl(t.off, 0), qbl = 0, fl = 0;
    for (int i = 0; i < t.nlev; ++i) {
        const int oi = rl(t.off, i), fi = rl(t.first, i);
        if (x >= oi + fi) koff = oi;  // K/V row base of level i
        if (t.lam_min + i >= t.lo) {
            const int qi = rl(t.qb, i);
            if (x >= qi) {
                qbl = qi;
                fl = fi;
            }
        }
    }
    const int sq = x - qbl;
    const int nd = divide(sq, gdiv);
    int kvnode = x - koff;                                        // K/V row x: node, relative to the tile's kv base
    if constexpr (PAGED) {
        const int lp = divide(kvnode, p.pdiv);  // kvnode >= 0
        kvnode = (lp << kSlotBits) | (kvnode - lp * p.page_size);
    }
    const int qpack = ((fl + nd) << 8) | (sq - nd * p.group);     // Q row x: node << 8 | q head in the group
    const int rsub = (threadIdx.x + z) / Geo::CPR;
#pragma unroll
    for (int ps = 0; ps < Geo::PASSES; ++ps) {
        const int r = ps * Geo::RPP + rsub;  // < 64
        rm.kvrow[ps] = lane_get(kvnode, r);
        rm.qrow[ps] = lane_get(qpack, r);  // group <= Q_ROWS (a plan exists)
    }
}

// Issue the global loads of a tile into the staging registers.
// PAGED: node x of the sequence lives in slot x % page_size of page
// pt[seq][x / page_size] (src/ragged_attn.py:822-929); pt_lds is the
// workgroup's LDS copy of the page table, in which a page outside
// [0, num_pages) reads -1.  A row whose logical page is past pt_cols or
// whose page is missing gets flag 0 in rowok (this
// tile's half of the double buffer; the compute masks the row out) and reads
// the tile's first Q row instead (in bounds, and finite whenever an output
// can be: P = 0 multiplies its V, the mask replaces its score).  Loads stay
// unconditional (a guarded load made the compiler keep a staged register in
// scratch and wait for it at issue), and the flags go to LDS at once, so
// nothing extra stays in registers across the compute of the previous tile.
template <int D, bool BATCH, bool PAGED>
__device__ __forceinline__ void tile_issue(const TreeParams& p, const TileMeta& t, const RowMap<D>& rm,
                                           Stage<D>& sg, const int32_t* pt_lds, int32_t* rowok) {
    using Geo = StreamGeom<D>;
    const int rsub = threadIdx.x / Geo::CPR;
    // (paged: z = 0 from the tile, so the per-lane base pointers below are
    // formed here rather than kept in registers across the loop)
    const int z = PAGED ? (t.nlev >> 7) : 0;
    const int c8 = 8 * ((threadIdx.x + z) % Geo::CPR);
    const int64_t kvb = PAGED ? 0 : t.kvb;
    const uint16_t* kg = (const uint16_t*)p.k + (kvb * p.sk_t + (int64_t)t.kvh * p.sk_h + c8);
    const uint16_t* vg = (const uint16_t*)p.v + (kvb * p.sv_t + (int64_t)t.kvh * (PAGED ? p.sk_h : p.sv_h) + c8);
    const uint16_t* qg =
        (const uint16_t*)p.q +
        ((int64_t)t.start * p.sq_t + (BATCH ? (int64_t)t.seq * p.sq_b : 0) + (int64_t)t.kvh * p.group * p.sq_h + c8);
    if constexpr (PAGED) {
        const int32_t* ptrow = pt_lds + t.seq * p.pt_cols;
        const bool c0 = (threadIdx.x % Geo::CPR) == 0;
#pragma unroll
        for (int ps = 0; ps < Geo::PASSES; ++ps) {
            if (ps * Geo::RPP >= t.rows) break;  // wave-uniform
            const int r = ps * Geo::RPP + rsub;
            if (r < t.rows) {
                const int32_t lp = rm.kvrow[ps] >> kSlotBits;
                const int32_t slot = rm.kvrow[ps] & ((1 << kSlotBits) - 1);
                const int32_t pg = lp < p.pt_cols ? ptrow[lp] : -1;
                const bool ok = pg >= 0;
                if (c0) rowok[r] = ok ? 1 : 0;
                const uint64_t off = (uint64_t)(uint32_t)pg * (uint32_t)p.sk_page +
                                     (uint64_t)(uint32_t)slot * (uint32_t)p.sk_t;
                const uint16_t* kr = ok ? kg + off : qg;
                const uint16_t* vr = ok ? vg + off : qg;
                sg.k[ps] = ld16(kr);
                sg.v[ps] = ld16(vr);
            }
        }
    } else {
#pragma unroll
        for (int ps = 0; ps < Geo::PASSES; ++ps) {
            if (ps * Geo::RPP >= t.rows) break;  // wave-uniform
            if (ps * Geo::RPP + rsub < t.rows) {
                sg.k[ps] = ld16(kg + (int64_t)rm.kvrow[ps] * p.sk_t);
                sg.v[ps] = ld16(vg + (int64_t)rm.kvrow[ps] * p.sv_t);
            }
        }
    }
#pragma unroll
    for (int ps = 0; ps < Geo::PASSES; ++ps) {
        if (ps * Geo::RPP >= t.nq) break;  // wave-uniform
        if (ps * Geo::RPP + rsub < t.nq)
            sg.q[ps] = ld16(qg + (int64_t)(rm.qrow[ps] >> 8) * p.sq_t + (int64_t)(rm.qrow[ps] & 255) * p.sq_h);
    }
}

// Write the staged tile to LDS (K, V and Q rows at the padded pitch).  V rows
// past the tile's last row keep the previous tile's (finite) values or the
// zeros written at kernel start; P = 0 multiplies them.
template <int D, bool DBG = false, bool PAGED = false>
__device__ __forceinline__ void tile_store(const TreeParams& p, const TileMeta& t, uint16_t* Ks, uint16_t* Vs,
                                           uint16_t* Qs, const Stage<D>& sg, const RowMap<D>& rm, int32_t* dbg_row,
                                           int32_t* dbg_q) {
    using Geo = StreamGeom<D>;
    const int tid = threadIdx.x;
    const int rsub = tid / Geo::CPR, c = tid % Geo::CPR;
    if constexpr (DBG) {
        // the map the loads of this tile were issued with (row r of LDS holds
        // node dbg_row[r] of the sequence; Q row q holds token/head dbg_q[q])
        if (c == 0) {
#pragma unroll
            for (int ps = 0; ps < Geo::PASSES; ++ps) {
                const int r = ps * Geo::RPP + rsub;
                dbg_row[r] = r < t.rows ? (PAGED ? (rm.kvrow[ps] >> kSlotBits) * p.page_size +
                                                       (rm.kvrow[ps] & ((1 << kSlotBits) - 1))
                                                 : rm.kvrow[ps])
                                        : -1;
                dbg_q[r] = r < t.nq ? rm.qrow[ps] : -1;
            }
        }
    }
#pragma unroll
    for (int ps = 0; ps < Geo::PASSES; ++ps) {
        if (ps * Geo::RPP >= t.rows) break;
        const int r = ps * Geo::RPP + rsub;
        if (r < t.rows) {
            st16(Ks + r * Geo::PITCH + 8 * c, sg.k[ps]);
            st16(Vs + r * Geo::PITCH + 8 * c, sg.v[ps]);
        }
    }
#pragma unroll
    for (int ps = 0; ps < Geo::PASSES; ++ps) {
        if (ps * Geo::RPP >= t.nq) break;
        const int q = ps * Geo::RPP + rsub;
        if (q < t.nq) st16(Qs + q * Geo::PITCH + 8 * c, sg.q[ps]);
    }
}

// Four 16-bit elements of V^T through the transposing LDS load: within each
// 16-lane group, lane j reads V[key0 + j / 4][d0 + 4 (j % 4) .. +3] and lane
// i receives V[key0 + k][d0 + i] for k = 0..3.
__device__ __forceinline__ uint2 vt_read4(const uint16_t* Vs, int pitch, int key0, int d0, int j) {
    typedef short v4s __attribute__((ext_vector_type(4)));
    const uint16_t* a = Vs + (key0 + (j >> 2)) * pitch + d0 + 4 * (j & 3);
    const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)a);
    return __builtin_bit_cast(uint2, r);
}

// Build the query table of a tile: the calling threads take queries q0,
// q0 + step, ... (q0 < step, one query per thread and pass).  The walk
// (src/ragged_attn.py:338-377) attends steps t = 0..min(level, max_depth),
// levels level - t, exactly the steps with c_t != c_{t-1}; the level loop runs
// from the deepest level up so every level offset is a wave-uniform readlane.
__device__ __forceinline__ void build_query_table(const TreeParams& p, const Divider& gdiv, const TileMeta& t,
                                                  QueryEntry* qt, int q0, int step) {
    const int g = p.group;
    for (int qs = 0; qs < t.nq; qs += step) {
        const int q = qs + q0;
        int li = -1, qbl = 0, fi = 0;
        for (int i = 0; i < t.nlev; ++i) {
            const int qi = rl(t.qb, i), ci = rl(t.cnt, i) * g, f = rl(t.first, i);
            if (t.lam_min + i >= t.lo && q >= qi && q < qi + ci) {
                li = i;
                qbl = qi;
                fi = f;
            }
        }
        const int s_in = q - qbl;
        const int nd = divide(s_in, gdiv);
        const int node = fi + nd;
        const int lam = t.lam_min + li;
        int steps = li >= 0 ? (lam < p.max_depth ? lam : p.max_depth) + 1 : 0;
        uint64_t mask = 0;
        int32_t cur = node;
        int lv = li;
        for (int i = t.nlev - 1; i >= 0; --i) {
            const int oi = rl(t.off, i);
            if (lv == i && steps > 0) {
                mask |= uint64_t(1) << (cur + oi);
                cur = heap_parent(cur, p.bdiv);
                --lv;
                --steps;
            }
        }
        if (q < t.nq) qt[q] = QueryEntry{(uint32_t)mask, (uint32_t)(mask >> 32), node, s_in - nd * g};
    }
}

// Walk export: the ancestor set each query of the tile attends, read back
// from what the compute uses -- its row mask in the query table, each set bit
// mapped to the node whose K/V row the loads put in that LDS row -- and
// written as [token][q head][step] (step = the query's depth minus the
// row's).  A bit on a row without a node, two rows at one step, or a Q row
// staged from another token/head than the table says marks the entry -2 at
// step 0.  vmask: the rows the compute keeps (paged K/V: rows with a page).
__device__ __forceinline__ void dbg_walk_export(const TreeParams& p, const TileMeta& t, const QueryEntry* qt,
                                                const int32_t* dbg_row, const int32_t* dbg_q, uint64_t vmask) {
    const int S1 = p.max_depth + 1;
    auto depth = [&](int32_t x) {
        int dd = 0;
        while (x > 0) {
            x = heap_parent(x, p.bdiv);
            ++dd;
        }
        return dd;
    };
    for (int q = threadIdx.x; q < t.nq; q += kStThreads) {
        const QueryEntry qe = qt[q];
        const uint64_t mask = (((uint64_t)qe.mask_hi << 32) | qe.mask_lo) & vmask;
        bool bad = dbg_q[q] != ((qe.node << 8) | qe.hoff);
        int32_t* out = p.dbg_walk + (((int64_t)t.start + qe.node) * p.Hq + t.kvh * p.group + qe.hoff) * S1;
        for (int i = 0; i < S1; ++i) out[i] = -1;
        const int dq = depth(qe.node);
        uint64_t filled = 0;
        for (int r = 0; r < 64; ++r) {
            if (!((mask >> r) & 1u)) continue;
            const int32_t node = dbg_row[r];
            const int step = node >= 0 ? dq - depth(node) : -1;
            if (node < 0 || step < 0 || step >= S1 || ((filled >> step) & 1u)) {
                bad = true;
                continue;
            }
            filled |= uint64_t(1) << step;
            out[step] = node;
        }
        if (bad) out[0] = -2;
    }
}

// One wave: attention of 16 queries (query block qb) of the tile held in LDS.
// vmask: the K/V rows that exist (all of them but paged rows without a page).
template <typename T, int D, bool LSE, bool PSTATE, bool BATCH>
__device__ __forceinline__ void block_compute(const TreeParams& p, const TileMeta& t, int qb, const uint16_t* Ks,
                                              const uint16_t* Vs, const uint16_t* Qs, const QueryEntry* qt,
                                              uint64_t vmask) {
    using Geo = StreamGeom<D>;
    constexpr int NC = Geo::NC, ND = Geo::ND, KT = Geo::KT;
    const int lane = threadIdx.x & 63;
    const int c16 = lane & 15, i4 = lane >> 4;
    const int g = p.group;

    // ---- this lane's query (column c16 of the block) ----
    const int sq = 16 * qb + c16;
    const bool qvalid = sq < t.nq;
    QueryEntry qe = QueryEntry{0u, 0u, 0, 0};
    if (qvalid) qe = qt[sq];
    const uint64_t mask = (((uint64_t)qe.mask_hi << 32) | qe.mask_lo) & vmask;
    const int64_t qrow = (int64_t)t.start + qe.node;
    const int qh = t.kvh * g + qe.hoff;

    // ---- S^T = K Q^T ----
    // Every key tile of the LDS buffer is multiplied (rows past the tile hold
    // stale but finite data or whatever LDS held; the row mask below selects
    // -inf for them).  Software-pipelined: the K operand of step i + 1 is read
    // before the product of step i is issued, and consecutive products
    // accumulate into different key tiles.
    Vec16 qf[NC];
#pragma unroll
    for (int kc = 0; kc < NC; ++kc) qf[kc] = ld16(Qs + (16 * qb + c16) * Geo::PITCH + 32 * kc + 8 * i4);
    f4_t sacc[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) sacc[kt] = f4_t{0.f, 0.f, 0.f, 0.f};
    {
        constexpr int NS = KT * NC;  // step i: kc = i / KT, kt = i % KT
        Vec16 kb[2];
        kb[0] = ld16(Ks + c16 * Geo::PITCH + 8 * i4);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if (i + 1 < NS) {
                const int kc1 = (i + 1) / KT, kt1 = (i + 1) % KT;
                kb[(i + 1) & 1] = ld16(Ks + (16 * kt1 + c16) * Geo::PITCH + 32 * kc1 + 8 * i4);
            }
            sacc[i % KT] = MfmaOps<T>::mma(kb[i & 1], qf[i / KT], sacc[i % KT]);
        }
    }

    __builtin_amdgcn_sched_barrier(0);  // keep the PV operand reads below the softmax
    // ---- masked softmax per query column ----
    // Scores are scaled before the mask and the max, so any finite scale
    // works (zero or negative included).
    const float c = p.scale_log2;
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const uint32_t bits = (uint32_t)(mask >> (16 * kt + 4 * i4)) & 15u;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float s = ((bits >> r) & 1u) ? sacc[kt][r] * c : -INFINITY;
            sacc[kt][r] = s;
            mx = fmaxf(mx, s);
        }
    }
    mx = col4_max(mx);
    float mref = (mx == -INFINITY) ? 0.f : mx;  // a query with no row (invalid column)
    // Split-K prefix partial states (flash-decoding merge): the reference
    // becomes max(tree max, prefix max) and the accumulators start from the
    // prefix states weighted by 2^(m_s - reference), one split at a time.
    float lpre = 0.f;
    f4_t oacc[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) oacc[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (PSTATE) {
        if (qvalid) {
            const int64_t plane = p.total_tokens * (int64_t)p.Hq;
            const int64_t idx = qrow * p.Hq + qh;
            float mp = -INFINITY;
            for (int s = 0; s < p.n_split; ++s) mp = fmaxf(mp, p.part_m[s * plane + idx]);
            if (mp != -INFINITY) {
                mref = fmaxf(mref, mp);
                for (int s = 0; s < p.n_split; ++s) {
                    const float ms = p.part_m[s * plane + idx];
                    if (ms == -INFINITY) continue;
                    // the split's numerator is stored as acc / l (kPartHalf)
                    const float wl = fast_exp2(ms - mref) * p.part_l[s * plane + idx];
                    lpre += wl;
                    const int64_t off = (s * plane + idx) * D + 4 * i4;
#pragma unroll
                    for (int dt = 0; dt < ND; ++dt) {
                        float4 v;
                        if constexpr (kPartHalf<T>) {
                            const uint2 h = *reinterpret_cast<const uint2*>((const uint16_t*)p.part_acc + off + 16 * dt);
                            v = make_float4(MfmaOps<F16>::lo(h.x), MfmaOps<F16>::hi(h.x), MfmaOps<F16>::lo(h.y),
                                            MfmaOps<F16>::hi(h.y));
                        } else {
                            v = *reinterpret_cast<const float4*>((const float*)p.part_acc + off + 16 * dt);
                        }
                        oacc[dt][0] = __builtin_fmaf(wl, v.x, oacc[dt][0]);
                        oacc[dt][1] = __builtin_fmaf(wl, v.y, oacc[dt][1]);
                        oacc[dt][2] = __builtin_fmaf(wl, v.z, oacc[dt][2]);
                        oacc[dt][3] = __builtin_fmaf(wl, v.w, oacc[dt][3]);
                    }
                }
            }
        }
    }
    const float mc = mref;
    float ls = 0.f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = fast_exp2(sacc[kt][r] - mc);  // -inf -> 0
            sacc[kt][r] = e;
            ls += e;
        }
    }
    ls = col4_sum(ls);

    // ---- O^T = V^T P^T, P = hi + lo in T ----
    // O is normalised after the product: P keeps its largest element at 1, so
    // the lo halves of the large elements stay fp16 normals (the products
    // lose subnormal fp16 inputs: normalising P first was measured to cost up
    // to 2e-3 relative in O)
    // Key tiles 2kk and 2kk+1 form the 32-key operands of 16x16x32 products;
    // an odd last key tile (48-row tiles) is a 16x16x16 product.
    constexpr int KF = KT / 2;        // 32-key chunks
    constexpr bool KTAIL = KT & 1;    // one 16-key chunk
    uint32_t ph[KT][2], pl[KT][2];    // P hi / lo of key tile kt, packed pairs
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float x = sacc[kt][2 * h], y = sacc[kt][2 * h + 1];
            const uint32_t w = MfmaOps<T>::pack2(x, y);
            ph[kt][h] = w;
            pl[kt][h] = MfmaOps<T>::pack2(x - MfmaOps<T>::lo(w), y - MfmaOps<T>::hi(w));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // All V_ROWS rows take part (P = 0 past the tile; those rows hold finite
    // values).  Software-pipelined like S: step i = (chunk, dt), chunk = i / ND,
    // reads its V^T operand one step ahead.
    {
        constexpr int NS = (KF + (KTAIL ? 1 : 0)) * ND;
        // A[d][e] of chunk kk: e = 0..3 -> key 32 kk + 4 i4 + e, e = 4..7 -> key
        // 32 kk + 16 + 4 i4 + (e - 4); the 16-key tail: e = 0..3 -> key 32 KF + 4 i4 + e
        uint2 va[2], vb[2];
        auto fetch = [&](int i, uint2& x, uint2& y) {
            const int kk = i / ND, dt = i % ND;
            x = vt_read4(Vs, Geo::PITCH, 32 * kk + 4 * i4, 16 * dt, c16);
            if (kk < KF) y = vt_read4(Vs, Geo::PITCH, 32 * kk + 16 + 4 * i4, 16 * dt, c16);
        };
        fetch(0, va[0], vb[0]);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if (i + 1 < NS) fetch(i + 1, va[(i + 1) & 1], vb[(i + 1) & 1]);
            const int kk = i / ND, dt = i % ND;
            if (kk < KF) {
                const Vec16 a = Vec16{{va[i & 1].x, va[i & 1].y, vb[i & 1].x, vb[i & 1].y}};
                const Vec16 bh = Vec16{{ph[2 * kk][0], ph[2 * kk][1], ph[2 * kk + 1][0], ph[2 * kk + 1][1]}};
                const Vec16 bl = Vec16{{pl[2 * kk][0], pl[2 * kk][1], pl[2 * kk + 1][0], pl[2 * kk + 1][1]}};
                oacc[dt] = MfmaOps<T>::mma(a, bh, oacc[dt]);
                oacc[dt] = MfmaOps<T>::mma(a, bl, oacc[dt]);
            } else {
                oacc[dt] = MfmaOps<T>::mma16(va[i & 1], make_uint2(ph[KT - 1][0], ph[KT - 1][1]), oacc[dt]);
                oacc[dt] = MfmaOps<T>::mma16(va[i & 1], make_uint2(pl[KT - 1][0], pl[KT - 1][1]), oacc[dt]);
            }
        }
    }

    // ---- normalise ----
    const float m = mc, l = ls + lpre;
    const float l_safe = (l == 0.f) ? 1.f : l;  // src/ragged_attn.py:379-380
    const float inv = __builtin_amdgcn_rcpf(l_safe);
    if constexpr (LSE) {
        // a query that attends nothing (paged rows without a page) has
        // m = -inf in the reference's formula
        if (qvalid && i4 == 0)
            p.lse[qrow * p.slse_t + (BATCH ? (int64_t)t.seq * p.slse_b : 0) + (int64_t)qh * p.slse_h] =
                l == 0.f ? -INFINITY : (m + fast_log2(l_safe)) * kLn2;
    }

    // ---- O: lane holds O^T[16 dt + 4 i4 + r][c16], stored straight as 8-byte
    // pieces; the 4 lanes of a column fill 32 contiguous bytes per d-tile and
    // the d-tiles complete the row in L2 ----
    if (qvalid) {
        uint16_t* optr =
            (uint16_t*)p.o + qrow * p.so_t + (BATCH ? (int64_t)t.seq * p.so_b : 0) + (int64_t)qh * p.so_h + 4 * i4;
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
            *reinterpret_cast<uint2*>(optr + 16 * dt) =
                make_uint2(MfmaOps<T>::pack2(oacc[dt][0] * inv, oacc[dt][1] * inv),
                           MfmaOps<T>::pack2(oacc[dt][2] * inv, oacc[dt][3] * inv));
        }
    }
}

template <typename T, int D, bool LSE, bool PSTATE, bool BATCH>
__device__ __forceinline__ void tile_compute(const TreeParams& p, const TileMeta& t, const uint16_t* Ks,
                                             const uint16_t* Vs, const uint16_t* Qs, const QueryEntry* qt,
                                             uint64_t vmask) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int qb = wave; 16 * qb < t.nq; qb += kStThreads / 64)
        block_compute<T, D, LSE, PSTATE, BATCH>(p, t, qb, Ks, Vs, Qs, qt, vmask);
}

// Next item of a group: one returning atomic on the group's counter.
__device__ __forceinline__ uint32_t sched_grab(uint32_t* ctr) {
    return __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The staging registers of one tile stay live across the compute phase of the
// previous one; 3 workgroups of 256 threads per CU (about 50 KB of LDS each)
// need at most 168 VGPRs.
//
// Schedule (StreamArgs): workgroup j of group g takes item j first.  With
// counters, thread 0 asks for the next item while the loads of the current
// one are in flight, and the answer is waited for with those loads, so the
// counter's latency is hidden; workgroups that started late or ran slow take
// fewer items.  Every workgroup that took part adds one to the group's done
// counter after its last request, and the last of them clears both counters,
// so the next launch finds them at zero.
// BATCH: a uniform batch (null cu, per-sequence q/o/lse offsets); the packed
// layout compiles without that addressing.
// DBG: the walk-export instantiation (qattn_debug_walk), which also writes
// every query's attended ancestor set to p.dbg_walk.
// PAGED: K/V rows from the paged cache through p.page_table (copied to LDS at
// kernel start; the host launches this only for B * pt_cols <= kPtCache).
template <typename T, int D, bool LSE, bool PSTATE, bool BATCH, bool DBG = false, bool PAGED = false>
__global__ __launch_bounds__(kStThreads)
__attribute__((amdgpu_waves_per_eu(3, 3))) void tree_stream_kernel(
    TreeParams p, SubtreePlan plan, StreamArgs sa) {
    using Geo = StreamGeom<D>;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    uint16_t* Ks = smem;
    uint16_t* Qs = Ks + Geo::KV_ROWS * Geo::PITCH;
    uint16_t* Vs = Qs + Geo::Q_ROWS * Geo::PITCH;
    // two query tables: the compute reads the current tile's while the next
    // tile's is built (a tile of another shape)
    QueryEntry* qtab = reinterpret_cast<QueryEntry*>(Vs + Geo::V_ROWS * Geo::PITCH);
    int32_t* cuc = reinterpret_cast<int32_t*>(qtab + 2 * Geo::Q_ROWS);
    int32_t* next_slot = cuc + kCuCache;  // the workgroup's next item, written by thread 0
    int32_t* lvl_lds = next_slot + 4;     // plan.lvl_start[0..63], plan.lvl_pow[0..63]
    int32_t* dbg_row = lvl_lds + 128;     // (DBG only: LDS_BYTES + DBG_BYTES are allocated)
    int32_t* dbg_q = dbg_row + Geo::KV_ROWS;
    // (PAGED only: ROWOK_BYTES + 4 B * B * pt_cols more are allocated; tile
    // flags alternate between the two halves of rowok, par selects the half
    // of the tile being computed)
    int32_t* rowok = dbg_row + (DBG ? Geo::KV_ROWS + Geo::Q_ROWS : 0);
    int32_t* pt_lds = rowok + 2 * Geo::KV_ROWS;
    int par = 0;
    const Divider gdiv = sa.gdiv;
    if constexpr (PAGED) {
        // the page table, before anything else: the first tile's loads need it
        // (the barrier below the first tile's setup publishes it); missing
        // pages become -1 here, once, so the tile loop does not test them.
        // (Staging these loads in registers, or issuing four before the
        // stores, measured slower.)
        const int npt = p.B * p.pt_cols;
        for (int i = threadIdx.x; i < npt; i += kStThreads) {
            const int32_t e = p.page_table[i];
            pt_lds[i] = (uint32_t)e < (uint32_t)p.num_pages ? e : -1;
        }
    }

    const int grp = divide((int)blockIdx.x, sa.ngroups);
    const int g = (int)blockIdx.x - grp * sa.ngroups.d;  // group
    // current item; grp < gsize <= items (the host's grid), so every workgroup
    // has a first item and no kernel argument has to arrive before the loads
    // below are addressed
    int k = grp;
    const bool dyn = sa.sched != nullptr;
    uint32_t* grab_ctr = dyn ? sa.sched + (size_t)g * kSchedStride : nullptr;
    uint32_t* done_ctr = dyn ? grab_ctr + 1 : nullptr;
    const bool leader = threadIdx.x == 0;
    // ans: the answer of this workgroup's last counter request (one variable,
    // so it stays in one register while the request is in flight)
    uint32_t ans = 0;
    const int w = k * sa.ngroups.d + g;
    // the plan's band table, one band per lane, from a single vector load
    // each: the scalar lookup took two dependent kernel-argument round trips
    // on every workgroup's first tile (~3.8 us at kernel start), and scalar
    // loads of the first 8 bands (one round trip) finished the first setup
    // 0.5 us later than these loads
    const int lane = threadIdx.x & 63;
    const int32_t band_tb = lane < kMaxBands ? plan.tile_base[lane] : INT32_MAX;
    const uint32_t band_pk = lane < kMaxBands ? plan.band[lane] : 0u;
    // the level tables of the first tile's setup, loaded with the band table
    const int32_t lvl_st0 = plan.lvl_start[lane];
    const uint32_t lvl_pw0 = plan.lvl_pow[lane];
    // V rows the PV product reads but no tile has written yet must hold finite
    // values (P = 0 multiplies them): zero them once.  Each thread zeroes the
    // V chunks it stages itself, so its own tile stores follow the zeros in
    // program order (the first loop top's barrier publishes both).
    {
        const int rsub = threadIdx.x / Geo::CPR, c = threadIdx.x % Geo::CPR;
#pragma unroll
        for (int ps = 0; ps < Geo::PASSES; ++ps)
            st16(Vs + (ps * Geo::RPP + rsub) * Geo::PITCH + 8 * c, Vec16{{0u, 0u, 0u, 0u}});
    }
    const int32_t __attribute__((address_space(3)))* cu_lds =
        (const int32_t __attribute__((address_space(3)))*)cuc;

    // The first tile takes the bounds of its sequence from wave-uniform
    // loads, and the LDS copy of cu_seqlens is written at the first loop top,
    // so nothing here waits for vector memory.
    TileMeta cur, none;
    none.valid = 0;
    int qcur = 0;  // the query table of the current tile
    RowMap<D> rm;
    Stage<D> sg;
    const int seq0 = tile_seq(sa, w);  // < p.B: w < n_work
    // (a uniform batch holds max_seqlen rows per sequence)
    const int32_t cu_mine = threadIdx.x > p.B ? 0
                            : BATCH        ? (int32_t)threadIdx.x * p.max_seqlen
                                           : p.cu[threadIdx.x];  // p.B < kCuCache = kStThreads
    const int32_t s0 = BATCH ? seq0 * p.max_seqlen : __builtin_amdgcn_readfirstlane(p.cu[seq0]);
    const int32_t e0 = BATCH ? s0 + p.max_seqlen : __builtin_amdgcn_readfirstlane(p.cu[seq0 + 1]);
    {
        const int tile0 = w - divide(w, sa.tiles_div) * plan.total_tiles;
        const int bi = (int)__builtin_popcountll(__ballot(tile0 >= band_tb)) - 1;
        const uint32_t bpk = (uint32_t)__builtin_amdgcn_readlane((int)band_pk, bi);
        const int tbase = __builtin_amdgcn_readlane(band_tb, bi);
        tile_setup_se<D, true>(p, plan, sa, w, s0, e0, none, cur, bpk, tbase, lvl_st0, lvl_pw0, lvl_lds);
    }
    // the level tables for later tiles' setups (published by the first loop top's barrier)
    if (threadIdx.x < 64) {
        lvl_lds[threadIdx.x] = lvl_st0;
        lvl_lds[64 + threadIdx.x] = (int32_t)lvl_pw0;
    }
    if constexpr (PAGED) __syncthreads();  // the LDS page table
    if (cur.valid) {
        tile_rowmap<D, PAGED>(p, gdiv, cur, rm);
        tile_issue<D, BATCH, PAGED>(p, cur, rm, sg, pt_lds, rowok);
        // the first query table is built while the first loads are in flight
        // (the first loop top's barrier publishes it)
        build_query_table(p, gdiv, cur, qtab, threadIdx.x, kStThreads);
    }
    if (dyn && leader) ans = sched_grab(grab_ctr);  // answered by the first loop top
    bool first = true;
    for (;;) {
        // The staged loads must have landed before they are written to LDS;
        // waiting for all vector memory here (the previous tile's O stores
        // have had a whole compute phase to drain) also means no path leaves
        // a load pending into the issue code below, which would otherwise get
        // a conservative wait on every outstanding store.
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        if (first && threadIdx.x <= p.B) cuc[threadIdx.x] = cu_mine;
        first = false;
        if (cur.valid) tile_store<D, DBG, PAGED>(p, cur, Ks, Vs, Qs, sg, rm, dbg_row, dbg_q);
        if (leader) *next_slot = dyn ? sa.gsize + (int)ans : k + sa.gsize;
        __syncthreads();
        const int kn = __builtin_amdgcn_readfirstlane(*next_slot);
        const bool more = kn < sa.items;
        const int wn = kn * sa.ngroups.d + g;
        TileMeta nxt;
        int qnxt = qcur;
        bool build = false;
        if (more) {
            const bool fresh = tile_setup<D>(p, plan, sa, cu_lds, wn, cur, nxt, band_tb, band_pk, lvl_lds);
            if (nxt.valid) {
                if (fresh) tile_rowmap<D, PAGED>(p, gdiv, nxt, rm);
                tile_issue<D, BATCH, PAGED>(p, nxt, rm, sg, pt_lds, rowok + (par ^ 1) * Geo::KV_ROWS);
                // the next tile's query table: the current one, or (another
                // shape) built into the other one after this compute
                build = !cur.valid || nxt.tile != cur.tile || nxt.n != cur.n;
                qnxt = build ? qcur ^ 1 : qcur;
            }
        }
        // the next item, or (after this workgroup's last request) done
        if (dyn && leader) ans = sched_grab(more ? grab_ctr : done_ctr);
        if (cur.valid) {
            const QueryEntry* qt = qtab + qcur * Geo::Q_ROWS;
            // the rows that exist: all, or (paged) those whose page does
            uint64_t vmask = ~uint64_t(0);
            if constexpr (PAGED) vmask = __ballot(lane < Geo::KV_ROWS && rowok[par * Geo::KV_ROWS + lane] != 0);
            if constexpr (DBG) dbg_walk_export(p, cur, qt, dbg_row, dbg_q, vmask);
            tile_compute<T, D, LSE, PSTATE, BATCH>(p, cur, Ks, Vs, Qs, qt, vmask);
        }
        // by the last wave, which computes the fewest query blocks (the
        // barrier below publishes it)
        if (build && threadIdx.x >= kStThreads - 64)
            build_query_table(p, gdiv, nxt, qtab + qnxt * Geo::Q_ROWS, lane, 64);
        __syncthreads();
        if (!more) break;
        cur = nxt;
        k = kn;
        par ^= 1;
        qcur = qnxt;
    }
    // The last workgroup of the group to finish clears its counters: every
    // other one has made its last request before adding to done_ctr.
    const int members = sa.items < sa.gsize ? sa.items : sa.gsize;
    if (dyn && leader && ans == (uint32_t)(members - 1)) {
        __hip_atomic_store(grab_ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(done_ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Scheduler counters (StreamArgs::sched): a static device array of
// kSchedGroups * kSchedStride words per device (each GPU holds its own copy),
// zeroed by qattn_init, holding kSchedSlots counter slots (a slot: one counter
// pair per group, kSchedStride words apart).  Every launch leaves its slot at
// zero when it completes.
//
// A slot may only serve launches that cannot overlap in time:
//  * an eager launch takes the slot of its stream (launches on one stream run
//    in order; the first kSchedStreamSlots streams seen on a device get one
//    each, later streams run the static schedule);
//  * launches recorded into a graph share one slot per (capture sequence,
//    capturing stream): they form a chain of the graph, which runs in order,
//    and replays of one graph executable run in order.  The slot goes back to
//    the pool when the graph and every executable made from it are destroyed
//    (a HIP user object that the graph retains; the runtime releases it once
//    the pending replays are done).  When the captured slots run out, the
//    launch is recorded with the static schedule.
// Before qattn_init has run on a device every launch uses the static schedule
// (same results, slower): the library never allocates, zeroes or
// synchronises behind a call.  qattn_sched_info reports the slots in use and
// how many launches ran each schedule.
constexpr int kSchedStreamSlots = 64, kSchedCapSlots = kSchedSlots - kSchedStreamSlots, kSchedMaxDev = 64;
static __device__ __align__(256) uint32_t sched_pool[kSchedGroups * kSchedStride];

namespace {
struct CapSlot {
    unsigned long long id = 0;  // capture sequence
    hipStream_t stream = nullptr;
    bool used = false;
};
struct SchedDevice {
    uint32_t* pool = nullptr;  // device address of this device's sched_pool
    hipStream_t streams[kSchedStreamSlots] = {};
    int n_streams = 0;
    CapSlot cap[kSchedCapSlots];
    int64_t dyn_launches = 0, static_launches = 0;
};
std::mutex g_sched_mu;
SchedDevice g_sched[kSchedMaxDev];

// What a captured slot's user object carries to its destructor.
struct CapToken {
    int dev, slot;
    unsigned long long id;
};

// Destructor of a captured slot's user object (run by the HIP runtime once
// the graph that retained it, and the executables made from it, are gone).
void release_cap_slot(void* arg) {
    CapToken* tk = static_cast<CapToken*>(arg);
    {
        std::lock_guard<std::mutex> lock(g_sched_mu);
        CapSlot& cs = g_sched[tk->dev].cap[tk->slot];
        if (cs.used && cs.id == tk->id) cs = CapSlot{};
    }
    delete tk;
}
}  // namespace

int sched_init(int dev) {
    if (dev < 0 || dev >= kSchedMaxDev) {
        set_error("device %d beyond the %d devices the library tracks", dev, kSchedMaxDev);
        return QATTN_ERR_ARG;
    }
    std::lock_guard<std::mutex> lock(g_sched_mu);
    if (g_sched[dev].pool) return QATTN_OK;
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(sched_pool)) != hipSuccess || !ptr) {
        set_error("hipGetSymbolAddress(sched_pool) failed on device %d", dev);
        return QATTN_ERR_HIP;
    }
    // zero the counters on a private stream (not the caller's, not captured)
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
        set_error("cannot create the init stream on device %d", dev);
        return QATTN_ERR_HIP;
    }
    const hipError_t e1 = hipMemsetAsync(ptr, 0, sizeof(sched_pool), s);
    const hipError_t e2 = hipStreamSynchronize(s);
    (void)hipStreamDestroy(s);
    if (e1 != hipSuccess || e2 != hipSuccess) {
        set_error("zeroing the schedule counters failed on device %d", dev);
        return QATTN_ERR_HIP;
    }
    g_sched[dev].pool = (uint32_t*)ptr;
    return QATTN_OK;
}

int sched_info(int dev, int64_t info[6]) {
    if (dev < 0 || dev >= kSchedMaxDev) {
        set_error("device %d beyond the %d devices the library tracks", dev, kSchedMaxDev);
        return QATTN_ERR_ARG;
    }
    std::lock_guard<std::mutex> lock(g_sched_mu);
    const SchedDevice& sd = g_sched[dev];
    int held = 0;
    for (const CapSlot& c : sd.cap) held += c.used ? 1 : 0;
    info[0] = sd.n_streams;
    info[1] = held;
    info[2] = sd.dyn_launches;
    info[3] = sd.static_launches;
    info[4] = kSchedStreamSlots;
    info[5] = kSchedCapSlots;
    return QATTN_OK;
}

// The counter slot of a launch on stream st, or null (static schedule).
static uint32_t* sched_counters(int dev, hipStream_t st) {
    if (dev < 0 || dev >= kSchedMaxDev) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    hipGraph_t graph = nullptr;
    if (hipStreamGetCaptureInfo_v2(st, &cs, &cid, &graph) != hipSuccess) return nullptr;
    const bool captured = cs != hipStreamCaptureStatusNone;
    if (captured && cs != hipStreamCaptureStatusActive) return nullptr;
    int slot = -1;
    bool fresh = false;
    uint32_t* pool = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_sched_mu);
        SchedDevice& sd = g_sched[dev];
        if (!sd.pool) return nullptr;
        pool = sd.pool;
        if (captured) {
            int free_slot = -1;
            for (int i = 0; i < kSchedCapSlots && slot < 0; ++i) {
                if (sd.cap[i].used && sd.cap[i].id == cid && sd.cap[i].stream == st) slot = i;
                else if (!sd.cap[i].used && free_slot < 0) free_slot = i;
            }
            if (slot < 0 && free_slot >= 0) {
                slot = free_slot;
                sd.cap[slot].used = true;
                sd.cap[slot].id = cid;
                sd.cap[slot].stream = st;
                fresh = true;
            }
            if (slot >= 0) slot += kSchedStreamSlots;
        } else {
            for (int i = 0; i < sd.n_streams; ++i)
                if (sd.streams[i] == st) slot = i;
            if (slot < 0 && sd.n_streams < kSchedStreamSlots) {
                slot = sd.n_streams++;
                sd.streams[slot] = st;
            }
        }
        if (slot < 0) {
            ++sd.static_launches;
            return nullptr;
        }
        ++sd.dyn_launches;
    }
    if (fresh) {
        // the graph being captured keeps the slot until it is destroyed (the
        // HIP calls run outside the lock: the destructor takes it).  Without
        // a user object the slot stays with this capture for the process's
        // life, which is still correct.
        CapToken* tk = new CapToken{dev, slot - kSchedStreamSlots, cid};
        hipUserObject_t obj = nullptr;
        if (hipUserObjectCreate(&obj, tk, release_cap_slot, 1, hipUserObjectNoDestructorSync) != hipSuccess) {
            delete tk;
        } else if (hipGraphRetainUserObject(graph, obj, 1, hipGraphUserObjectMove) != hipSuccess) {
            (void)hipUserObjectRelease(obj, 1);  // runs the destructor: frees the slot
            std::lock_guard<std::mutex> lock(g_sched_mu);
            --g_sched[dev].dyn_launches;
            ++g_sched[dev].static_launches;
            return nullptr;
        }
    }
    return pool + 2 * slot;
}

template <typename T, int D, bool LSE, bool PSTATE, bool BATCH, bool DBG = false, bool PAGED = false>
static int launch_stream_t(const TreeParams& p, const SubtreePlan& plan, hipStream_t st) {
    using Geo = StreamGeom<D>;
    const int64_t n_work = (int64_t)p.B * p.Hkv * plan.total_tiles;
    if (n_work >= (int64_t(1) << 31)) {
        set_error("too many subtree tiles (%lld)", (long long)n_work);
        return QATTN_ERR_ARG;
    }
    if (n_work == 0) return QATTN_OK;
    if (p.B >= kCuCache) {
        set_error("subtree kernel: batch %d exceeds %d sequences", p.B, kCuCache - 1);
        return QATTN_ERR_ARG;
    }
    const int64_t npt = PAGED ? (int64_t)p.B * p.pt_cols : 0;
    if (PAGED && (npt > kPtCache || !p.page_table || p.page_size < 1)) {
        set_error("subtree kernel: page table of %lld entries exceeds %d", (long long)npt, kPtCache);
        return QATTN_ERR_ARG;
    }
    const size_t lds = Geo::LDS_BYTES + (DBG ? Geo::DBG_BYTES : 0) +
                       (PAGED ? Geo::ROWOK_BYTES + (size_t)npt * 4 : 0);
    auto kern = tree_stream_kernel<T, D, LSE, PSTATE, BATCH, DBG, PAGED>;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kStThreads, lds) != hipSuccess) {
        set_error("cannot query the device for the subtree launch");
        return QATTN_ERR_HIP;
    }
    // a multiple of the tile count when possible: each workgroup then keeps one
    // tile index (its group) and reuses its level table across (sequence, kv
    // head) pairs; otherwise one group over all tiles
    const int64_t cap = (int64_t)std::max(cus, 1) * std::max(per_cu, 1);
    int64_t grid = std::min<int64_t>(n_work, cap);
    int64_t ngroups = 1;
    if (plan.total_tiles <= cap) {
        ngroups = plan.total_tiles;
        grid = std::max<int64_t>(1, std::min<int64_t>(n_work, cap) / ngroups) * ngroups;
    }
    StreamArgs sa;
    sa.n_work = (int32_t)n_work;
    sa.tiles_div = make_divider(plan.total_tiles);
    sa.hkv_div = make_divider(p.Hkv);
    sa.gdiv = make_divider(p.group);
    sa.ngroups = make_divider((int32_t)ngroups);
    sa.gsize = (int32_t)(grid / ngroups);
    sa.items = (int32_t)(n_work / ngroups);
    if (sa.gsize > sa.items) {  // not for this grid: every workgroup needs a first item
        set_error("subtree launch: %d workgroups per group for %d items", sa.gsize, sa.items);
        return QATTN_ERR_ARG;
    }
    sa.sched = (ngroups <= kSchedGroups && sa.items > sa.gsize) ? sched_counters(dev, st) : nullptr;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kStThreads), lds, st, p, plan, sa);
    return launch_status("tree_stream_kernel");
}

// Walk export (qattn_debug_walk): the walk-export instantiation of the
// kernel that serves the same call (dtype, LSE, prefix state, paged K/V).
template <typename T, int D>
static int launch_stream_dbg(const TreeParams& p, const SubtreePlan& plan, bool pstate, bool paged,
                             hipStream_t st) {
    if (p.lse) {
        if (paged) return launch_stream_t<T, D, true, false, false, true, true>(p, plan, st);
        return pstate ? launch_stream_t<T, D, true, true, false, true>(p, plan, st)
                      : launch_stream_t<T, D, true, false, false, true>(p, plan, st);
    }
    if (paged) return launch_stream_t<T, D, false, false, false, true, true>(p, plan, st);
    return pstate ? launch_stream_t<T, D, false, true, false, true>(p, plan, st)
                  : launch_stream_t<T, D, false, false, false, true>(p, plan, st);
}

int launch_stream(const TreeParams& p, const SubtreePlan& plan, int dtype, int head_dim, bool pstate, bool paged,
                  hipStream_t st) {
    if (paged && (pstate || !p.cu)) {
        set_error("the paged subtree kernel takes packed cu_seqlens and no prefix state");
        return QATTN_ERR_ARG;
    }
    if (p.dbg_walk) {
        // walk export: calls over packed cu_seqlens, either dtype, with or without LSE
        if (!p.cu) {
            set_error("the walk export runs calls over packed cu_seqlens");
            return QATTN_ERR_ARG;
        }
        if (dtype == QATTN_DTYPE_F16)
            return head_dim == 32   ? launch_stream_dbg<F16, 32>(p, plan, pstate, paged, st)
                   : head_dim == 64 ? launch_stream_dbg<F16, 64>(p, plan, pstate, paged, st)
                                    : launch_stream_dbg<F16, 128>(p, plan, pstate, paged, st);
        return head_dim == 32   ? launch_stream_dbg<BF16, 32>(p, plan, pstate, paged, st)
               : head_dim == 64 ? launch_stream_dbg<BF16, 64>(p, plan, pstate, paged, st)
                                : launch_stream_dbg<BF16, 128>(p, plan, pstate, paged, st);
    }
#define QATTN_STREAM_B(T, D, B)                                                                \
    if (p.lse) return pstate ? launch_stream_t<T, D, true, true, B>(p, plan, st)                \
                             : launch_stream_t<T, D, true, false, B>(p, plan, st);              \
    return pstate ? launch_stream_t<T, D, false, true, B>(p, plan, st)                          \
                  : launch_stream_t<T, D, false, false, B>(p, plan, st);
#define QATTN_STREAM_D(T, D)                                                                   \
    if (paged) return p.lse ? launch_stream_t<T, D, true, false, false, false, true>(p, plan, st)   \
                            : launch_stream_t<T, D, false, false, false, false, true>(p, plan, st); \
    if (!p.cu) { QATTN_STREAM_B(T, D, true) }                                                     \
    QATTN_STREAM_B(T, D, false)
    if (dtype == QATTN_DTYPE_F16) {
        if (head_dim == 32) { QATTN_STREAM_D(F16, 32) }
        if (head_dim == 64) { QATTN_STREAM_D(F16, 64) }
        QATTN_STREAM_D(F16, 128)
    }
    if (head_dim == 32) { QATTN_STREAM_D(BF16, 32) }
    if (head_dim == 64) { QATTN_STREAM_D(BF16, 64) }
    QATTN_STREAM_D(BF16, 128)
#undef QATTN_STREAM_D
#undef QATTN_STREAM_B
}

}  // namespace qattn
