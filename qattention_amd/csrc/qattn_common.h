// qattn_common.h -- host/device shared definitions: parameter blocks, the
// heap-walk divider, the subtree tiling plan and error reporting.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qattn.h"

namespace qattn {

// ---------------------------------------------------------------------------
// Division by the branching factor.  The heap walk needs
// parent(c) = max(c - 1, 0) / b  (src/ragged_attn.py:376-377, clamp before the
// divide).  b is a launch constant, so the divide becomes a multiply-high:
// with l = ceil(log2 b) and m = floor(2^32 (2^l - b) / b) + 1,
// x / b = (mulhi(x, m) + x) >> l for every 0 <= x < 2^31.
// ---------------------------------------------------------------------------
struct Divider {
    uint32_t magic;
    int32_t shift;
    int32_t d;
};

inline Divider make_divider(int32_t d) {
    Divider r;
    r.d = d;
    int l = 0;
    while ((int64_t(1) << l) < d) ++l;
    r.shift = l;
    uint64_t num = (uint64_t(1) << 32) * ((uint64_t(1) << l) - uint64_t(d));
    r.magic = uint32_t(num / uint64_t(d) + 1);
    return r;
}

__device__ __forceinline__ int32_t divide(int32_t x, const Divider& dv) {
    uint32_t ux = uint32_t(x);
    uint32_t hi = __umulhi(ux, dv.magic);
    return int32_t((hi + ux) >> dv.shift);
}

// One step of the heap ancestor walk: max(c - 1, 0) / b.
__device__ __forceinline__ int32_t heap_parent(int32_t c, const Divider& dv) {
    int32_t m = c - 1;
    m = m > 0 ? m : 0;
    return divide(m, dv);
}

// ---------------------------------------------------------------------------
// Parameter block of the tree kernels (passed by value as a kernel argument).
// Strides are in elements; the d-stride of every tensor is 1.
// ---------------------------------------------------------------------------
struct TreeParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    const int32_t* cu;          // [B+1] sequence offsets into q/o (and packed k/v); null: uniform
                                // batch, sequence s holds rows [s * max_seqlen, (s + 1) * max_seqlen)
    const int32_t* parents;     // explicit-parent walk: sequence-local parent per token
    const int32_t* page_table;  // paged K/V: [B, pt_cols] physical page per logical page
    int64_t sq_t, sq_h, sk_t, sk_h, sv_t, sv_h, so_t, so_h;
    int64_t slse_t, slse_h;
    int64_t sk_page, sv_page;   // paged K/V: elements between pages (sk_t/sv_t = slot stride)
    int64_t total_tokens;       // rows of q / o
    int64_t kv_rows;            // rows of packed k / v
    int32_t num_pages, pt_cols, page_size;
    int32_t B, Hq, Hkv, group, max_seqlen, max_depth;
    Divider bdiv;               // branching factor
    Divider pdiv;               // paged K/V: page_size
    Divider hqdiv, msdiv;       // Hq and max_seqlen (>= 1): the gather kernel's slot decomposition
    float scale_log2;           // softmax scale * log2(e)
    // split-K prefix partial state merged into the tree state (may be null)
    const float* part_m;        // [n_split][T][Hq]   running max (log2 domain)
    const float* part_l;        // [n_split][T][Hq]   running denominator
    const void* part_acc;       // [n_split][T][Hq][D] numerator / l: fp16 for fp16 inputs, else fp32
    int32_t n_split;
    // tree K/V location of sequence `seq` is cu[seq] + kv_seq_off * seq
    // (0 for the packed layout; the hybrid layout places L prefix rows before
    // every sequence's tree rows).
    int64_t kv_row0;            // extra row offset before the tree rows of each sequence
    int64_t kv_seq_stride;      // rows between consecutive sequences in k/v (0: use cu)
    // Uniform batch only (null cu; kept last so the packed layout's fields
    // keep their kernel-argument offsets): per-sequence element offsets added
    // to the q / o / lse address of every row of sequence s (times s), and the
    // parents of sequence s start at index s * par_stride (0: one array shared
    // by every sequence; packed: at the sequence's first row).
    int64_t sq_b, so_b, slse_b;
    int32_t par_stride;
    // Walk export (qattn_debug_walk; null in normal calls): int32
    // [total_tokens][Hq][max_depth + 1], entry i = the node a query attended
    // at walk step i, or -1.  Only the kernels' debug instantiations read it.
    int32_t* dbg_walk;
};

// Subtree tiling of a heap-indexed tree (levels of the BFS order).
constexpr int kMaxBands = 32;
struct Band {
    int32_t lo, hi, G, tile_base;
};
// Kernel argument form of the plan: the band of a tile is found with one
// branch-free pass over tile_base[] (independent scalar loads) and one more
// load of its packed (lo, hi, G).
struct SubtreePlan {
    int32_t nbands;
    int32_t total_tiles;
    int32_t max_rows;                 // LDS rows (K and V each) of the largest tile
    int32_t chain_h;                  // b == 1: levels per tile
    int32_t tile_base[kMaxBands];     // first tile of band i; INT32_MAX past the last band
    uint32_t band[kMaxBands];         // lo | hi << 8 | G << 16
    // Heap level tables for l = 0..63: lvl_start[l] = (b^l - 1) / (b - 1),
    // the first node of BFS level l (INT32_MAX once it passes that), and
    // lvl_pow[l] = b^l (UINT32_MAX once it passes that); b == 1: l and 1.
    // Descendants j levels below node x start at x * b^j + lvl_start[j], and
    // the ancestor k levels above x is (x - lvl_start[k]) / b^k.
    int32_t lvl_start[64];
    uint32_t lvl_pow[64];
};

// Launch arguments of the persistent subtree kernel (subtree_stream.hip).
// Work items of the subtree kernel: item k of group g is tile index
// w = k * ngroups + g (w as in the comment of tile_setup).  Workgroup
// blockIdx = j * ngroups + g starts with item j; with sched set, later items
// come from the group's counter pair (sched[g * kSchedStride] hands out items
// gsize, gsize+1, ...; sched[g * kSchedStride + 1] counts the workgroups that
// are done, and the last one resets both to zero), without it workgroup j
// takes j, j + gsize, ...  Counter pairs of one launch lie kSchedStride words
// (2 KB) apart, so no two groups share a cache line: atomics on one line are
// serialised, and 4000-8000 requests per launch on a single line made the
// kernel 10-20% slower.  The words in between hold other slots' pairs.  A
// launch has at most 3 workgroups per CU, so at most 768 groups on 256 CUs.
constexpr int kSchedGroups = 1024;
constexpr int kSchedSlots = 256;                // launches with counters of their own
constexpr int kSchedStride = 2 * kSchedSlots;   // words between groups of one launch

struct StreamArgs {
    int32_t n_work;     // tiles over all (sequence, kv head) pairs
    Divider tiles_div;  // tiles per (sequence, kv head)
    Divider hkv_div;    // kv heads
    Divider gdiv;       // q heads per kv head
    Divider ngroups;    // work groups
    int32_t gsize;      // workgroups per group (grid = gsize * ngroups)
    int32_t items;      // items per group (n_work = items * ngroups)
    uint32_t* sched;    // the launch's counter pairs (zero), or null (static schedule)
};

// Subtree kernel: rows one tile may stage (K/V rows, Q rows) for head_dim,
// the largest batch it takes (its LDS copy of cu_seqlens) and, for paged K/V,
// the largest page table (B * pt_cols entries, copied to LDS).
void stream_tile_caps(int head_dim, int* kv_rows, int* q_rows);
int stream_max_batch();
int stream_max_page_entries();
// paged: K/V through p.page_table (heap walk, no prefix state)
int launch_stream(const TreeParams& p, const SubtreePlan& plan, int dtype, int head_dim, bool pstate, bool paged,
                  hipStream_t st);
// qattn_init's part for the subtree kernel: the device address of the
// current device's counter pool, zeroed (synchronously, on a private stream).
int sched_init(int dev);
// qattn_sched_info's figures for device dev (see include/qattn.h).
int sched_info(int dev, int64_t info[6]);

void set_error(const char* fmt, ...);
void clear_error();

// Host helpers shared by the entry points (tree_attn.hip).  fill_tree_params
// with uniform set takes a null cu (every sequence holds max_seqlen rows).
bool row_aligned(const void* ptr, const int64_t* st, int n_outer);
int check_common(int32_t dtype, int32_t head_dim, int32_t batch, int32_t max_seqlen, int64_t total_tokens,
                 int32_t hq, int32_t hkv, int32_t max_depth);
int launch_status(const char* what);
int fill_tree_params(TreeParams& p, const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                     const void* v, const int64_t* vs, void* o, const int64_t* os, float* lse, const int64_t* lss,
                     const int32_t* cu, int32_t batch, int32_t max_seqlen, int64_t total_tokens, int32_t hq,
                     int32_t hkv, int32_t b, int32_t max_depth, float scale, bool uniform = false);
// walk: 0 heap, 1 parents; layout: 0 packed, 1 paged
int run_tree(const TreeParams& p, int dtype, int head_dim, int walk, int layout, bool pstate, int algo,
             hipStream_t st);

}  // namespace qattn
