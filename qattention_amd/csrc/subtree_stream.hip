// subtree_stream.hip -- persistent, software-pipelined subtree kernel for the
// heap ancestor walk (src/ragged_attn.py:262-387 over complete b-ary heaps).
//
// The heap parent (i-1)/b makes the ancestors of a subtree a union of
// contiguous BFS level ranges, so the host cuts each tree into tiles (a band
// of levels under G adjacent roots, plus one ancestor row per level above the
// band; make_subtree_plan in tree_attn.hip).  Every K/V row of a tile is read
// from HBM once per kv head, and every ancestor read of every query in the
// tile is an LDS read.
//
// Each workgroup is persistent and walks tiles w, w + gridDim.x, ...  One tile
// is always in flight: right after tile i is written to LDS, the workgroup
// computes the metadata of tile i+1 and issues its global loads (K and V rows
// of the tile, and the Q rows of its queries) into registers, then computes
// tile i from LDS.  The loads of tile i+1 land while tile i is computed, so
// HBM sees a steady stream of requests instead of each workgroup's
// load-wait-compute phases.  Q is staged through LDS with K and V, so the
// compute phase never waits on global memory; O is written straight from
// registers.
//
// Compute: a query is owned by 8 lanes (4 for D = 32), each owning one
// contiguous slice of the row (32 bytes at D = 128), so a wave walks 8 queries
// of one BFS level at a time with a wave-uniform step count; every ancestor
// step is one LDS row read for K and V, a v_dot2 chain + DPP sum for the score
// and v_fma_mix for the V accumulation, with a lazily moved softmax
// reference.  LDS rows are D + 8 elements apart (one 16-byte pad chunk).
#include <algorithm>

#include "qattn_common.h"
#include "qattn_device.h"
#include "tree_walk.h"

namespace qattn {

constexpr int kStThreads = 256;
constexpr int kKVPass = 3;    // K/V staging passes per tile (2 vectors each)
constexpr int kQPass = 3;     // Q staging passes per tile (1 vector each)
constexpr float kLazy = 8.f;    // softmax reference moves only past 2^kLazy
constexpr int kCuCache = 256;   // cu_seqlens entries cached in LDS

template <int D>
struct StreamGeom {
    static constexpr int CPR = D / 8;               // 16-byte chunks per row
    static constexpr int PITCH = D + 8;             // LDS row pitch in elements
    static constexpr int ROWS_PER_PASS = kStThreads / CPR;
    static constexpr int KV_ROWS = kKVPass * ROWS_PER_PASS;  // max K/V rows per tile
    static constexpr int Q_ROWS = kQPass * ROWS_PER_PASS;    // max Q rows per tile
    static constexpr int LPQ = D >= 64 ? 8 : 4;     // lanes per query
    static constexpr int NCH = CPR / LPQ;           // 16-byte chunks per lane (contiguous)
    static constexpr int QPW = 64 / LPQ;            // queries per wave item
};

// Per-tile state.  Scalars are wave-uniform; first/cnt/off/qb are per lane,
// lane i describing BFS level lam_min + i.
struct TileMeta {
    int32_t valid, tile, seq, kvh, start, n, lo, hi, lam_min, nlev, rows, nq;
    int64_t kvb;
    int32_t first, cnt, off, qb;
};

// Per-thread source rows of the staging passes of a tile: K/V pass ps reads
// node (row - offr[ps]); Q pass ps reads query (row - qbl[ps]) of the level
// whose first node is fl[ps].  Depends only on the level table, so it is
// reused while a workgroup stays on the same tile; it lives in LDS (each
// thread reads back only its own entries), not in registers.
constexpr int kRowMapInts = kKVPass + 2 * kQPass;
typedef int32_t __attribute__((address_space(3))) * lds_i32_ptr;

int stream_max_batch() { return kCuCache - 1; }

void stream_tile_caps(int head_dim, int* kv_rows, int* q_rows) {
    const int rpp = kStThreads / (head_dim / 8);
    *kv_rows = kKVPass * rpp;
    *q_rows = kQPass * rpp;
}

// Which tile w is, and its level table (src/ragged_attn.py:376-377 walk:
// the ancestors of roots r0..r1-1 at level lo are, per level, one contiguous
// node range).  Returns true when the level table was (re)computed, false
// when it was taken from prev (same tile index and sequence length).
template <int D>
__device__ __forceinline__ bool tile_setup(const TreeParams& p, const SubtreePlan& plan, const StreamArgs& sa,
                                           const int32_t __attribute__((address_space(3)))* cu_lds, int w,
                                           const TileMeta& prev, TileMeta& t) {
    const int lane = threadIdx.x & 63;
    t.valid = 0;
    t.rows = t.nq = 0;
    t.nlev = 0;
    t.lo = 0;
    t.hi = -1;
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
    // cu_seqlens from the workgroup's LDS copy (the host launches this kernel
    // only for B < kCuCache): a global load here would make the wait for it
    // also wait for every O store still in flight.  readfirstlane: the offsets
    // are wave-uniform, so every tile scalar derived from them stays in SGPRs
    // and every branch on them is a scalar branch.
    const int32_t s = __builtin_amdgcn_readfirstlane(cu_lds[seq]);
    const int32_t e = __builtin_amdgcn_readfirstlane(cu_lds[seq + 1]);
    if (s < 0 || e < s || (int64_t)e > p.total_tokens) return true;
    int32_t n = e - s;
    if (n > p.max_seqlen) n = p.max_seqlen;
    if (n <= 0) return true;
    if (prev.valid && prev.tile == tile && prev.n == n) {
        t = prev;
        t.tile = tile;
        t.seq = seq;
        t.kvh = pair - seq * p.Hkv;
        t.start = s;
        t.kvb = kv_base(p, seq, s);
        return false;
    }
    const int b = p.bdiv.d;

    int bi = 0;
#pragma unroll
    for (int i = 1; i < kMaxBands; ++i) bi += (tile >= plan.tile_base[i]) ? 1 : 0;
    const uint32_t bpk = plan.band[bi];
    int lo = (int)(bpk & 255u), hi = (int)((bpk >> 8) & 255u);
    const int G = (int)(bpk >> 16), tbase = plan.tile_base[bi];
    int64_t r0, r1;  // root range [r0, r1) at level lo
    if (b == 1) {
        lo = (tile - tbase) * plan.chain_h;
        hi = lo + plan.chain_h - 1;
        r0 = lo;
        r1 = lo + 1;
    } else {
        int64_t s_lo = 0, w_lo = 1;
        for (int i = 0; i < lo; ++i) {
            s_lo += w_lo;
            w_lo *= b;
        }
        const int64_t i0 = (int64_t)(tile - tbase) * G;
        r0 = s_lo + i0;
        r1 = s_lo + ((i0 + G < w_lo) ? i0 + G : w_lo);
    }
    if (r0 >= n) return true;
    if (r1 > n) r1 = n;

    const int lam_min = (lo - p.max_depth > 0) ? lo - p.max_depth : 0;
    const int nlev = hi - lam_min + 1;  // <= 64, guaranteed by the host plan
    int first = 0, cnt = 0;
    const int lam = lam_min + lane;
    if (lane < nlev) {
        int64_t f, la;
        if (lam >= lo) {
            const int jj = lam - lo;
            int64_t bj = 1, sj = 0;
            for (int i = 0; i < jj; ++i) {
                sj += bj;
                bj *= b;
            }
            f = r0 * bj + sj;
            la = r1 * bj + sj - 1;
        } else {
            int32_t a = (int32_t)r0, c = (int32_t)(r1 - 1);
            for (int i = 0; i < lo - lam; ++i) {
                a = heap_parent(a, p.bdiv);
                c = heap_parent(c, p.bdiv);
            }
            f = a;
            la = c;
        }
        if (la > n - 1) la = n - 1;
        if (f <= la) {
            first = (int)f;
            cnt = (int)(la - f + 1);
        }
    }
    // exclusive prefix sums over levels: K/V LDS row base, Q LDS row base
    const int qc = (lane < nlev && lam >= lo) ? cnt * p.group : 0;
    int base = 0, qb = 0;
    for (int i = 0; i < nlev; ++i) {
        const int c = rl(cnt, i), cq = rl(qc, i);
        base += (i < lane) ? c : 0;
        qb += (i < lane) ? cq : 0;
    }
    const int rows = rl(base + cnt, nlev - 1);
    const int nq = rl(qb + qc, nlev - 1);
    if (rows > StreamGeom<D>::KV_ROWS || nq > StreamGeom<D>::Q_ROWS) return true;  // not for a host-built plan
    t.start = s;
    t.n = n;
    t.lo = lo;
    t.hi = hi;
    t.lam_min = lam_min;
    t.nlev = nlev;
    t.rows = rows;
    t.nq = nq;
    t.kvb = kv_base(p, seq, s);
    t.first = first;
    t.cnt = cnt;
    t.off = base - first;
    t.qb = qb;
    t.valid = 1;
    return true;
}

// Source rows of this thread's staging passes (K/V pass ps covers K/V rows
// [ps * RPP, (ps + 1) * RPP), Q pass ps Q rows likewise, RPP = rows per pass;
// thread tid handles chunk tid % CPR of row tid / CPR).
template <int D>
__device__ __forceinline__ void tile_rowmap(const TileMeta& t, lds_i32_ptr rmap) {
    using Geo = StreamGeom<D>;
    const int rsub = threadIdx.x / Geo::CPR;
    struct {
        int32_t offr[kKVPass], qbl[kQPass], fl[kQPass];
    } rm;
#pragma unroll
    for (int ps = 0; ps < kKVPass; ++ps) rm.offr[ps] = rl(t.off, 0);
#pragma unroll
    for (int ps = 0; ps < kQPass; ++ps) {
        rm.qbl[ps] = 0;
        rm.fl[ps] = 0;
    }
    for (int i = 0; i < t.nlev; ++i) {
        const int ci = rl(t.cnt, i);
        if (ci == 0) continue;
        const int oi = rl(t.off, i), fi = rl(t.first, i);
        const int bi = oi + fi, qi = rl(t.qb, i);
#pragma unroll
        for (int ps = 0; ps < kKVPass; ++ps) {
            if (ps * Geo::ROWS_PER_PASS + rsub >= bi) rm.offr[ps] = oi;
        }
        if (t.lam_min + i >= t.lo) {
#pragma unroll
            for (int ps = 0; ps < kQPass; ++ps) {
                if (ps * Geo::ROWS_PER_PASS + rsub >= qi) {
                    rm.qbl[ps] = qi;
                    rm.fl[ps] = fi;
                }
            }
        }
    }
    const int tid = threadIdx.x;
#pragma unroll
    for (int ps = 0; ps < kKVPass; ++ps) rmap[ps * kStThreads + tid] = rm.offr[ps];
#pragma unroll
    for (int ps = 0; ps < kQPass; ++ps) {
        rmap[(kKVPass + ps) * kStThreads + tid] = rm.qbl[ps];
        rmap[(kKVPass + kQPass + ps) * kStThreads + tid] = rm.fl[ps];
    }
}

// Issue the global loads of a tile into the staging registers.
template <int D>
__device__ __forceinline__ void tile_issue(const TreeParams& p, const Divider& gdiv, const TileMeta& t,
                                           lds_i32_ptr rmap, Vec16 (&kv)[kKVPass][2], Vec16 (&qv)[kQPass]) {
    using Geo = StreamGeom<D>;
    const int tid = threadIdx.x;
    const int rsub = tid / Geo::CPR, c = tid % Geo::CPR;
    const uint16_t* kg = (const uint16_t*)p.k + (int64_t)t.kvh * p.sk_h + 8 * c;
    const uint16_t* vg = (const uint16_t*)p.v + (int64_t)t.kvh * p.sv_h + 8 * c;
#pragma unroll
    for (int ps = 0; ps < kKVPass; ++ps) {
        if (ps * Geo::ROWS_PER_PASS >= t.rows) break;  // wave-uniform
        const int r = ps * Geo::ROWS_PER_PASS + rsub;
        if (r < t.rows) {
            const int64_t row = t.kvb + (r - rmap[ps * kStThreads + tid]);
            kv[ps][0] = ld16(kg + row * p.sk_t);
            kv[ps][1] = ld16(vg + row * p.sv_t);
        }
    }
    const int g = p.group;
#pragma unroll
    for (int ps = 0; ps < kQPass; ++ps) {
        if (ps * Geo::ROWS_PER_PASS >= t.nq) break;  // wave-uniform
        const int q = ps * Geo::ROWS_PER_PASS + rsub;
        if (q < t.nq) {
            const int sq = q - rmap[(kKVPass + ps) * kStThreads + tid];
            const int nd = divide(sq, gdiv);
            const int node = rmap[(kKVPass + kQPass + ps) * kStThreads + tid] + nd;
            const int head = t.kvh * g + (sq - nd * g);
            qv[ps] = ld16((const uint16_t*)p.q + ((int64_t)t.start + node) * p.sq_t + (int64_t)head * p.sq_h + 8 * c);
        }
    }
}

template <int D>
__device__ __forceinline__ void tile_store(const TileMeta& t, uint16_t* Ks, uint16_t* Vs, uint16_t* Qs,
                                           const Vec16 (&kv)[kKVPass][2], const Vec16 (&qv)[kQPass]) {
    using Geo = StreamGeom<D>;
    const int tid = threadIdx.x;
    const int rsub = tid / Geo::CPR, c = tid % Geo::CPR;
#pragma unroll
    for (int ps = 0; ps < kKVPass; ++ps) {
        if (ps * Geo::ROWS_PER_PASS >= t.rows) break;
        const int r = ps * Geo::ROWS_PER_PASS + rsub;
        if (r < t.rows) {
            st16(Ks + r * Geo::PITCH + 8 * c, kv[ps][0]);
            st16(Vs + r * Geo::PITCH + 8 * c, kv[ps][1]);
        }
    }
#pragma unroll
    for (int ps = 0; ps < kQPass; ++ps) {
        if (ps * Geo::ROWS_PER_PASS >= t.nq) break;
        const int q = ps * Geo::ROWS_PER_PASS + rsub;
        if (q < t.nq) st16(Qs + q * Geo::PITCH + 8 * c, qv[ps]);
    }
}

// q . k of one query against one LDS row (lane j of the query's LPQ lanes
// owns elements [8 NCH j, 8 NCH (j+1)) of every row): one dependent chain of
// v_dot2 per lane, then a DPP sum over the query's lanes.
template <typename T, int NCH, int LPQ>
__device__ __forceinline__ float qk_row(const Vec16* qf, const Vec16* kf) {
    float d = dot2<T>(qf[0].w[0], kf[0].w[0], 0.f);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
#pragma unroll
        for (int w = (i == 0 ? 1 : 0); w < 4; ++w) d = dot2<T>(qf[i].w[w], kf[i].w[w], d);
    }
    return group_sum<LPQ>(d);
}

// Initial state from split-K prefix partials, contiguous lane layout (lane j
// of a query owns elements [8 NCH j, 8 NCH (j+1))).
template <int D>
__device__ __forceinline__ void load_partial_state_c(const TreeParams& p, int64_t qrow, int h, int j, float& m,
                                                     float& l, float* acc) {
    constexpr int NCH = StreamGeom<D>::NCH;
    const int64_t plane = p.total_tokens * (int64_t)p.Hq;
    const int64_t idx = qrow * p.Hq + h;
    float m0 = -INFINITY;
    for (int s = 0; s < p.n_split; ++s) m0 = fmaxf(m0, p.part_m[s * plane + idx]);
    m = m0;
    l = 0.f;
#pragma unroll
    for (int e = 0; e < 8 * NCH; ++e) acc[e] = 0.f;
    if (m0 == -INFINITY) return;
    for (int s = 0; s < p.n_split; ++s) {
        const float ms = p.part_m[s * plane + idx];
        if (ms == -INFINITY) continue;
        const float w = fast_exp2(ms - m0);
        l = __builtin_fmaf(w, p.part_l[s * plane + idx], l);
        const float* a = p.part_acc + (s * plane + idx) * D + 8 * NCH * j;
#pragma unroll
        for (int e = 0; e < 8 * NCH; e += 4) {
            const float4 v = *reinterpret_cast<const float4*>(a + e);
            acc[e] = __builtin_fmaf(w, v.x, acc[e]);
            acc[e + 1] = __builtin_fmaf(w, v.y, acc[e + 1]);
            acc[e + 2] = __builtin_fmaf(w, v.z, acc[e + 2]);
            acc[e + 3] = __builtin_fmaf(w, v.w, acc[e + 3]);
        }
    }
}

// Normalise and store one query's output, contiguous lane layout (+ LSE).
template <typename T, int D, bool LSE>
__device__ __forceinline__ void write_out_c(const TreeParams& p, int64_t qrow, int h, int j, float m, float l,
                                            float* acc) {
    constexpr int NCH = StreamGeom<D>::NCH;
    const float l_safe = (l == 0.f) ? 1.f : l;  // src/ragged_attn.py:379-380
    const float inv = __builtin_amdgcn_rcpf(l_safe);
    uint16_t* optr = (uint16_t*)p.o + qrow * p.so_t + (int64_t)h * p.so_h + 8 * NCH * j;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = acc[8 * i + e] * inv;
        st16(optr + 8 * i, pack8<T>(r));
    }
    if constexpr (LSE) {
        if (j == 0) p.lse[qrow * p.slse_t + (int64_t)h * p.slse_h] = (m + fast_log2(l_safe)) * kLn2;
    }
}

template <typename T, int D, bool LSE, bool PSTATE>
__device__ __forceinline__ void tile_compute(const TreeParams& p, const Divider& gdiv, const TileMeta& t,
                                             const uint16_t* Ks, const uint16_t* Vs, const uint16_t* Qs) {
    using Geo = StreamGeom<D>;
    constexpr int NCH = Geo::NCH, LPQ = Geo::LPQ, QPW = Geo::QPW;
    const int lane64 = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane64 / LPQ, j = lane64 % LPQ;
    const int g = p.group;
    // wave items: QPW (node, q head) pairs of one level; item k of level L
    const int lam_l = t.lam_min + lane64;
    const int nw = (lane64 < t.nlev && lam_l >= t.lo) ? (t.cnt * g + QPW - 1) / QPW : 0;
    int L = t.lo, k = wave;
    for (;;) {
        while (L <= t.hi) {
            const int w = rl(nw, L - t.lam_min);
            if (k < w) break;
            k -= w;
            ++L;
        }
        if (L > t.hi) break;
        const int li = L - t.lam_min;
        const int s = k * QPW + grp;
        if (s < rl(t.cnt, li) * g) {
            const int nd = divide(s, gdiv);
            const int node = rl(t.first, li) + nd;
            const int qh = t.kvh * g + (s - nd * g);
            const int64_t qrow = (int64_t)t.start + node;
            Vec16 qf[NCH];
            const uint16_t* qs = Qs + (rl(t.qb, li) + s) * Geo::PITCH + 8 * NCH * j;
#pragma unroll
            for (int i = 0; i < NCH; ++i) qf[i] = ld16(qs + 8 * i);
            // steps t = 0..min(L, max_depth) attend levels L - t: the heap walk
            // strictly decreases until the root, so these are exactly the
            // steps with c_t != c_{t-1} (src/ragged_attn.py:338-377).
            const int nsteps = (L < p.max_depth ? L : p.max_depth) + 1;
            const float c = p.scale_log2;
            int32_t cur = node;
            int lv = li;  // level index (lane of the level table) of cur
            float m, l, acc[8 * NCH];
            int t0 = 0;
            if constexpr (PSTATE) {
                load_partial_state_c<D>(p, qrow, qh, j, m, l, acc);
            } else {
                // step 0, the query's own row, sets the reference: p = 1
                const int row = (cur + rl(t.off, lv)) * Geo::PITCH + 8 * NCH * j;
                Vec16 kf[NCH], vf[NCH];
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    kf[i] = ld16(Ks + row + 8 * i);
                    vf[i] = ld16(Vs + row + 8 * i);
                }
                m = qk_row<T, NCH, LPQ>(qf, kf) * c;
                l = 1.f;
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[8 * i + e] = elem<T>(vf[i], e);
                }
                cur = heap_parent(cur, p.bdiv);
                --lv;
                t0 = 1;
            }
            // Lazy rescaling: the reference m moves only when a score exceeds
            // it by more than kLazy (log2 units), so P <= 2^kLazy and the
            // accumulators are rescaled on few steps; l shares the reference,
            // so o = acc / l and lse = m + log2(l) are unchanged.
            for (int st = t0; st < nsteps; ++st) {
                const int row = (cur + rl(t.off, lv)) * Geo::PITCH + 8 * NCH * j;
                Vec16 kf[NCH], vf[NCH];
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    kf[i] = ld16(Ks + row + 8 * i);
                    vf[i] = ld16(Vs + row + 8 * i);
                }
                const float sc = qk_row<T, NCH, LPQ>(qf, kf) * c;
                const bool move = sc > m + kLazy;
                if (__builtin_expect(__any(move), 0)) {
                    const float m_new = move ? sc : m;
                    const float alpha = fast_exp2(m - m_new);  // m = -inf (empty state): 0
                    l *= alpha;
#pragma unroll
                    for (int e = 0; e < 8 * NCH; ++e) acc[e] *= alpha;
                    m = m_new;
                }
                const float pt = fast_exp2(sc - m);
                l += pt;
#pragma unroll
                for (int i = 0; i < NCH; ++i) axpy8<T>(acc + 8 * i, pt, vf[i]);
                cur = heap_parent(cur, p.bdiv);
                --lv;
            }
            write_out_c<T, D, LSE>(p, qrow, qh, j, m, l, acc);
        }
        k += kStThreads / 64;
    }
}

// The staging registers of one tile stay live across the compute phase of the
// previous one; 3 workgroups of 256 threads per CU (about 49 KB of LDS each)
// need at most 168 VGPRs.
template <typename T, int D, bool LSE, bool PSTATE>
__global__ __launch_bounds__(kStThreads) __attribute__((amdgpu_waves_per_eu(3, 3))) void tree_stream_kernel(
    TreeParams p, SubtreePlan plan, StreamArgs sa) {
    using Geo = StreamGeom<D>;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    uint16_t* Ks = smem;
    uint16_t* Vs = Ks + Geo::KV_ROWS * Geo::PITCH;
    uint16_t* Qs = Vs + Geo::KV_ROWS * Geo::PITCH;
    int32_t* cuc = reinterpret_cast<int32_t*>(Qs + Geo::Q_ROWS * Geo::PITCH);
    const lds_i32_ptr rmap = (lds_i32_ptr)(cuc + kCuCache);
    const Divider gdiv = sa.gdiv;

    int w = blockIdx.x;
    if (w >= sa.n_work) return;  // uniform: no barrier below is skipped by a subset of waves
    for (int i = threadIdx.x; i <= p.B; i += kStThreads) cuc[i] = p.cu[i];  // p.B < kCuCache
    __syncthreads();
    const int32_t __attribute__((address_space(3)))* cu_lds =
        (const int32_t __attribute__((address_space(3)))*)cuc;

    TileMeta cur, none;
    none.valid = 0;
    tile_setup<D>(p, plan, sa, cu_lds, w, none, cur);
    Vec16 kv[kKVPass][2], qv[kQPass];
    if (cur.valid) {
        tile_rowmap<D>(cur, rmap);
        tile_issue<D>(p, gdiv, cur, rmap, kv, qv);
    }
    for (;;) {
        if (cur.valid) tile_store<D>(cur, Ks, Vs, Qs, kv, qv);
        __syncthreads();
        const int wn = w + gridDim.x;
        const bool more = wn < sa.n_work;
        TileMeta nxt;
        if (more) {
            const bool fresh = tile_setup<D>(p, plan, sa, cu_lds, wn, cur, nxt);
            if (nxt.valid) {
                if (fresh) tile_rowmap<D>(nxt, rmap);
                tile_issue<D>(p, gdiv, nxt, rmap, kv, qv);
            }
        }
        if (cur.valid) tile_compute<T, D, LSE, PSTATE>(p, gdiv, cur, Ks, Vs, Qs);
        __syncthreads();
        if (!more) break;
        cur = nxt;
        w = wn;
    }
}

template <typename T, int D, bool LSE, bool PSTATE>
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
    const size_t lds = ((size_t)2 * Geo::KV_ROWS + Geo::Q_ROWS) * Geo::PITCH * 2 + kCuCache * 4 +
                       (size_t)kRowMapInts * kStThreads * 4;
    auto kern = tree_stream_kernel<T, D, LSE, PSTATE>;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kStThreads, lds) != hipSuccess) {
        set_error("cannot query the device for the subtree launch");
        return QATTN_ERR_HIP;
    }
    // a multiple of the tile count when possible: each workgroup then keeps one
    // tile index and reuses its level table across (sequence, kv head) pairs
    const int64_t cap = (int64_t)std::max(cus, 1) * std::max(per_cu, 1);
    int64_t grid = std::min<int64_t>(n_work, cap);
    if (plan.total_tiles <= cap && grid < n_work) grid = cap / plan.total_tiles * plan.total_tiles;
    StreamArgs sa;
    sa.n_work = (int32_t)n_work;
    sa.tiles_div = make_divider(plan.total_tiles);
    sa.hkv_div = make_divider(p.Hkv);
    sa.gdiv = make_divider(p.group);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kStThreads), lds, st, p, plan, sa);
    return launch_status("tree_stream_kernel");
}

int launch_stream(const TreeParams& p, const SubtreePlan& plan, int dtype, int head_dim, bool pstate,
                  hipStream_t st) {
#define QATTN_STREAM_D(T, D)                                                                  \
    if (p.lse) return pstate ? launch_stream_t<T, D, true, true>(p, plan, st)                  \
                             : launch_stream_t<T, D, true, false>(p, plan, st);                \
    return pstate ? launch_stream_t<T, D, false, true>(p, plan, st) : launch_stream_t<T, D, false, false>(p, plan, st);
    if (dtype == QATTN_DTYPE_F16) {
        if (head_dim == 32) { QATTN_STREAM_D(F16, 32) }
        if (head_dim == 64) { QATTN_STREAM_D(F16, 64) }
        QATTN_STREAM_D(F16, 128)
    }
    if (head_dim == 32) { QATTN_STREAM_D(BF16, 32) }
    if (head_dim == 64) { QATTN_STREAM_D(BF16, 64) }
    QATTN_STREAM_D(BF16, 128)
#undef QATTN_STREAM_D
}

}  // namespace qattn
