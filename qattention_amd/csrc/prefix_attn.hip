// prefix_attn.hip -- MFMA flash attention of tree-verify queries over a prefix
// KV cache (the dense half of src/ragged_attn.py:1761-1798), split along the
// prefix (flash-decoding) and merged into the tree walk's softmax state.
//
// Work unit: (sequence, kv head, query tile of 64 rows, prefix split).  The 64
// rows of a tile are (token, q head) pairs of ONE kv head's GQA group, so a
// K/V block staged in LDS serves every q head that reads it (no repeat_kv).
// Each of the 4 waves owns 16 rows and computes, per 64-key block,
//   S^T = K Q^T            16 x v_mfma_f32_16x16x32_{f16,bf16}
//   O^T += V^T P^T         16 x v_mfma_f32_16x16x32_{f16,bf16}   (D = 128)
// Computing S transposed puts one query per lane column, so the softmax row
// statistics need only a 4-lane (xor 16, xor 32) reduction and the MFMA
// output of S^T is directly the B operand P^T of the next product (keys are
// permuted consistently in P^T and in the LDS copy of V^T).
// The split's unnormalised state (m, l, acc) is written to a caller-provided
// workspace; the tree kernels (tree_attn.hip) merge all splits, walk the
// ancestors and normalise.
#include <algorithm>

#include "qattn_common.h"
#include "qattn_device.h"

namespace qattn {

constexpr int kPrefixThreads = 256;
constexpr int kBN = 64;  // prefix keys per block
constexpr int kBM = 64;  // query rows per workgroup (4 waves x 16)

struct PrefixParams {
    const void* q;
    const void* kp;
    const void* vp;
    const int32_t* cu;
    float* part_m;
    float* part_l;
    float* part_acc;
    int64_t sq_t, sq_h;
    int64_t skp_b, skp_t, skp_h, svp_b, svp_t, svp_h;
    int64_t total_tokens;
    int32_t B, Hq, Hkv, group, max_seqlen, L;
    int32_t n_split, blocks_per_split, qtiles, n_units;
    Divider gdiv;
    float scale_log2;
};

template <typename T>
struct MfmaOps;

template <>
struct MfmaOps<F16> {
    static __device__ __forceinline__ f4_t mma(const Vec16& a, const Vec16& b, f4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0,
                                                     0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float x, float y) {
        h2_t h;
        h[0] = (_Float16)x;
        h[1] = (_Float16)y;
        return __builtin_bit_cast(uint32_t, h);
    }
};

template <>
struct MfmaOps<BF16> {
    static __device__ __forceinline__ f4_t mma(const Vec16& a, const Vec16& b, f4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0,
                                                      0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float x, float y) {
        b2_t h;
        h[0] = (__bf16)x;
        h[1] = (__bf16)y;
        return __builtin_bit_cast(uint32_t, h);
    }
};

__device__ __forceinline__ float xor_max(float x, int m) { return fmaxf(x, __shfl_xor(x, m)); }

// Column of key k (0..63) of a block in the LDS copy of V^T: within each 32-key
// half, key 16u + 4g + j sits at 8g + 4u + j, so the 8 keys a lane feeds to
// one PV MFMA (4 from each of two S^T tiles) are contiguous.
__device__ __forceinline__ int vt_col(int k) {
    const int half = k >> 5, r = k & 31;
    const int u = r >> 4, g = (r >> 2) & 3, j = r & 3;
    return 32 * half + 8 * g + 4 * u + j;
}

template <typename T, int D>
__global__ __launch_bounds__(kPrefixThreads) void prefix_splitk_kernel(PrefixParams p) {
    constexpr int NC = D / 32;      // MFMA k-chunks over the head dim
    constexpr int ND = D / 16;      // output tiles over the head dim
    constexpr int KROW = D + 8;     // Ks row stride in elements (16-byte pad)
    constexpr int VROW = kBN + 8;   // Vt row stride in elements
    constexpr int DV = D / 8;       // 16-byte vectors per head row
    __shared__ __attribute__((aligned(16))) uint16_t Ks[kBN * KROW];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VROW];

    // Logical unit order puts the query tiles of one (sequence, kv head, split)
    // next to each other; hardware deals blockIdx round-robin over the 8 XCDs,
    // so unit u runs on XCD (blockIdx % 8) and a K/V block is shared in one L2.
    const int per = gridDim.x >> 3;
    const int unit = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (unit >= p.n_units) return;
    const int qt = unit % p.qtiles;
    int r = unit / p.qtiles;
    const int split = r % p.n_split;
    r /= p.n_split;
    const int kvh = r % p.Hkv;
    const int seq = r / p.Hkv;

    const int32_t s0 = p.cu[seq], s1 = p.cu[seq + 1];
    if (s0 < 0 || s1 < s0 || (int64_t)s1 > p.total_tokens) return;
    int32_t n = s1 - s0;
    if (n > p.max_seqlen) n = p.max_seqlen;
    const int g = p.group;
    const int rows = n * g;
    if (qt * kBM >= rows) return;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int l16 = lane & 15;
    const int lq = lane >> 4;

    // this lane's query row (B operand column / output column)
    const int rr = qt * kBM + wave * 16 + l16;
    const bool rvalid = rr < rows;
    const int tok = rvalid ? divide(rr, p.gdiv) : 0;
    const int qh = kvh * g + (rr - divide(rr, p.gdiv) * g);
    const int64_t qrow = (int64_t)s0 + tok;

    Vec16 qf[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        qf[c] = Vec16{{0u, 0u, 0u, 0u}};
        if (rvalid) qf[c] = ld16((const uint16_t*)p.q + qrow * p.sq_t + (int64_t)qh * p.sq_h + 32 * c + 8 * lq);
    }

    const int k_lo = split * p.blocks_per_split * kBN;
    const int k_hi = (k_lo + p.blocks_per_split * kBN < p.L) ? k_lo + p.blocks_per_split * kBN : p.L;
    const uint16_t* kbase = (const uint16_t*)p.kp + (int64_t)seq * p.skp_b + (int64_t)kvh * p.skp_h;
    const uint16_t* vbase = (const uint16_t*)p.vp + (int64_t)seq * p.svp_b + (int64_t)kvh * p.svp_h;

    float m_run = -INFINITY, l_run = 0.f;
    f4_t oacc[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) oacc[i] = f4_t{0.f, 0.f, 0.f, 0.f};

    for (int kb = k_lo; kb < k_hi; kb += kBN) {
        // ---- stage K (row-major, padded) and V^T (column-permuted) in LDS ----
#pragma unroll
        for (int u = tid; u < kBN * DV; u += kPrefixThreads) {
            const int key = u / DV, ch = u % DV;
            Vec16 x = Vec16{{0u, 0u, 0u, 0u}};
            if (kb + key < k_hi) x = ld16(kbase + (int64_t)(kb + key) * p.skp_t + 8 * ch);
            st16(Ks + key * KROW + 8 * ch, x);
        }
#pragma unroll
        for (int u = tid; u < (kBN / 4) * DV; u += kPrefixThreads) {
            const int kg = u % (kBN / 4), dch = u / (kBN / 4);
            Vec16 v4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = kb + 4 * kg + i;
                v4[i] = Vec16{{0u, 0u, 0u, 0u}};
                if (key < k_hi) v4[i] = ld16(vbase + (int64_t)key * p.svp_t + 8 * dch);
            }
            const int col = vt_col(4 * kg);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                // d = 8 dch + 2m (low halves) and 8 dch + 2m + 1 (high halves)
                const uint32_t e01 = __builtin_amdgcn_perm(v4[1].w[m], v4[0].w[m], 0x05040100u);
                const uint32_t e23 = __builtin_amdgcn_perm(v4[3].w[m], v4[2].w[m], 0x05040100u);
                const uint32_t o01 = __builtin_amdgcn_perm(v4[1].w[m], v4[0].w[m], 0x07060302u);
                const uint32_t o23 = __builtin_amdgcn_perm(v4[3].w[m], v4[2].w[m], 0x07060302u);
                *reinterpret_cast<uint2*>(Vt + (8 * dch + 2 * m) * VROW + col) = make_uint2(e01, e23);
                *reinterpret_cast<uint2*>(Vt + (8 * dch + 2 * m + 1) * VROW + col) = make_uint2(o01, o23);
            }
        }
        __syncthreads();

        // ---- S^T = K Q^T: lane holds keys 16 mt + 4 lq + i of query l16 ----
        f4_t sacc[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            sacc[mt] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const Vec16 a = ld16(Ks + (16 * mt + l16) * KROW + 32 * c + 8 * lq);
                sacc[mt] = MfmaOps<T>::mma(a, qf[c], sacc[mt]);
            }
        }
        float s[4][4];
        float mb = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = kb + 16 * mt + 4 * lq + i;
                const float v = (key < k_hi) ? sacc[mt][i] * p.scale_log2 : -INFINITY;
                s[mt][i] = v;
                mb = fmaxf(mb, v);
            }
        }
        mb = xor_max(mb, 16);
        mb = xor_max(mb, 32);
        const float m_new = fmaxf(m_run, mb);
        const float alpha = fast_exp2(m_run - m_new);  // m_run = -inf on the first block: 0
        float psum = 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[mt][i] = fast_exp2(s[mt][i] - m_new);
                psum += s[mt][i];
            }
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) oacc[dt] *= alpha;

        // ---- O^T += V^T P^T, two 32-key chunks ----
        Vec16 pf[2];
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            pf[kc].w[0] = MfmaOps<T>::pack2(s[2 * kc][0], s[2 * kc][1]);
            pf[kc].w[1] = MfmaOps<T>::pack2(s[2 * kc][2], s[2 * kc][3]);
            pf[kc].w[2] = MfmaOps<T>::pack2(s[2 * kc + 1][0], s[2 * kc + 1][1]);
            pf[kc].w[3] = MfmaOps<T>::pack2(s[2 * kc + 1][2], s[2 * kc + 1][3]);
        }
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                const Vec16 a = ld16(Vt + (16 * dt + l16) * VROW + 32 * kc + 8 * lq);
                oacc[dt] = MfmaOps<T>::mma(a, pf[kc], oacc[dt]);
            }
        }
        __syncthreads();
    }

    // ---- partial state of this split: (m, l, unnormalised acc) ----
    float l_tot = l_run + __shfl_xor(l_run, 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (!rvalid) return;
    const int64_t plane = p.total_tokens * (int64_t)p.Hq;
    const int64_t idx = (int64_t)split * plane + qrow * p.Hq + qh;
    if (lq == 0) {
        p.part_m[idx] = m_run;
        p.part_l[idx] = l_tot;
    }
    float* dst = p.part_acc + idx * D + 4 * lq;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
        *reinterpret_cast<float4*>(dst + 16 * dt) = make_float4(oacc[dt][0], oacc[dt][1], oacc[dt][2], oacc[dt][3]);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int prefix_splits(int64_t units_per_split, int L, int num_splits, int& blocks_per_split) {
    const int blocks = (L + kBN - 1) / kBN;
    int s = num_splits;
    if (s <= 0) {
        // aim for ~4 workgroups per CU on 256 CUs
        s = (int)std::min<int64_t>(blocks, std::max<int64_t>(1, (1024 + units_per_split - 1) / units_per_split));
    }
    s = std::max(1, std::min(s, std::max(blocks, 1)));
    blocks_per_split = (blocks + s - 1) / s;
    return blocks_per_split > 0 ? (blocks + blocks_per_split - 1) / blocks_per_split : 1;
}

static int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

static int64_t workspace_bytes(int64_t total_tokens, int hq, int head_dim, int splits) {
    const int64_t plane = total_tokens * hq;
    return 2 * align256(splits * plane * 4) + align256(splits * plane * head_dim * 4);
}

static int64_t units_per_split(int batch, int hkv, int max_seqlen, int group) {
    const int64_t qtiles = ((int64_t)max_seqlen * group + kBM - 1) / kBM;
    return (int64_t)batch * hkv * qtiles;
}

template <typename T, int D>
static int launch_prefix(const PrefixParams& pp, hipStream_t st) {
    const int64_t grid = ((int64_t)pp.n_units + 7) / 8 * 8;
    if (grid >= (int64_t(1) << 31)) {
        set_error("prefix grid too large");
        return QATTN_ERR_ARG;
    }
    hipLaunchKernelGGL((prefix_splitk_kernel<T, D>), dim3((unsigned)grid), dim3(kPrefixThreads), 0, st, pp);
    return launch_status("prefix_splitk_kernel");
}

}  // namespace qattn

using namespace qattn;

extern "C" {

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
    int rc = check_common(dtype, head_dim, batch, max_seqlen, total_tokens, num_q_heads, num_kv_heads, max_depth);
    if (rc) return rc;
    if (prefix_len < 0 || tree_seq_stride < 0 || tree_row0 < 0) {
        set_error("bad prefix_len / tree layout (%d, %lld, %lld)", prefix_len, (long long)tree_seq_stride,
                  (long long)tree_row0);
        return QATTN_ERR_ARG;
    }
    if (batch == 0 || max_seqlen == 0 || total_tokens == 0) return QATTN_OK;
    TreeParams tp;
    rc = fill_tree_params(tp, q, q_stride, k, k_stride, v, v_stride, o, o_stride, lse, lse_stride, cu_seqlens, batch,
                          max_seqlen, total_tokens, num_q_heads, num_kv_heads, branching_factor, max_depth, scale);
    if (rc) return rc;
    if (!row_aligned(k, k_stride, 2) || !row_aligned(v, v_stride, 2)) {
        set_error("k/v rows must be 16-byte aligned with stride_dim 1");
        return QATTN_ERR_LAYOUT;
    }
    tp.kv_seq_stride = tree_seq_stride;
    tp.kv_row0 = tree_row0;
    hipStream_t st = (hipStream_t)stream;
    if (prefix_len == 0) return run_tree(tp, dtype, head_dim, 0, 0, false, QATTN_ALGO_AUTO, st);

    if (!k_prefix || !v_prefix || !kp_stride || !vp_stride) {
        set_error("prefix pointers are null");
        return QATTN_ERR_ARG;
    }
    if (((uintptr_t)k_prefix & 15) || ((uintptr_t)v_prefix & 15) || kp_stride[1] % 8 || kp_stride[2] % 8 ||
        vp_stride[1] % 8 || vp_stride[2] % 8 || kp_stride[0] % 8 || vp_stride[0] % 8) {
        set_error("prefix rows must be 16-byte aligned (strides in multiples of 8 elements)");
        return QATTN_ERR_LAYOUT;
    }
    const int g = num_q_heads / num_kv_heads;
    int bps = 0;
    const int64_t ups = units_per_split(batch, num_kv_heads, max_seqlen, g);
    const int splits = prefix_splits(ups, prefix_len, num_splits, bps);
    const int64_t need = workspace_bytes(total_tokens, num_q_heads, head_dim, splits);
    if (!workspace || workspace_size < need || ((uintptr_t)workspace & 255)) {
        set_error("workspace of %lld bytes (256-byte aligned) required, got %lld", (long long)need,
                  (long long)workspace_size);
        return QATTN_ERR_WORKSPACE;
    }
    if (ups * splits >= (int64_t(1) << 31)) {
        set_error("too many prefix work units");
        return QATTN_ERR_ARG;
    }
    const int64_t plane = total_tokens * num_q_heads;
    PrefixParams pp{};
    pp.q = q;
    pp.kp = k_prefix;
    pp.vp = v_prefix;
    pp.cu = cu_seqlens;
    pp.part_m = (float*)workspace;
    pp.part_l = (float*)((char*)workspace + align256(splits * plane * 4));
    pp.part_acc = (float*)((char*)workspace + 2 * align256(splits * plane * 4));
    pp.sq_t = q_stride[0];
    pp.sq_h = q_stride[1];
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
    pp.qtiles = (int32_t)(((int64_t)max_seqlen * g + kBM - 1) / kBM);
    pp.n_units = (int32_t)(ups * splits);
    pp.gdiv = make_divider(g);
    pp.scale_log2 = scale * kLog2e;
    if (dtype == QATTN_DTYPE_F16) {
        rc = head_dim == 32 ? launch_prefix<F16, 32>(pp, st)
             : head_dim == 64 ? launch_prefix<F16, 64>(pp, st)
                              : launch_prefix<F16, 128>(pp, st);
    } else {
        rc = head_dim == 32 ? launch_prefix<BF16, 32>(pp, st)
             : head_dim == 64 ? launch_prefix<BF16, 64>(pp, st)
                              : launch_prefix<BF16, 128>(pp, st);
    }
    if (rc) return rc;
    tp.part_m = pp.part_m;
    tp.part_l = pp.part_l;
    tp.part_acc = pp.part_acc;
    tp.n_split = splits;
    return run_tree(tp, dtype, head_dim, 0, 0, true, QATTN_ALGO_AUTO, st);
}

}  // extern "C"
