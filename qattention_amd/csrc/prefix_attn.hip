// prefix_attn.hip -- MFMA flash attention of tree-verify queries over a prefix
// KV cache (the dense half of src/ragged_attn.py:1761-1798), merged into the
// ancestor walk's softmax state.
//
// Work unit: (sequence, kv head, query tile of 128 rows, prefix split).  The
// rows of a tile are (token, q head) pairs of ONE kv head's GQA group, so a
// K/V block staged in LDS serves every q head that reads it (no repeat_kv).
// Each of the 4 waves owns 32 rows as two 16-column blocks and computes, per
// 64-key block,
//   S^T = K Q^T      32 x v_mfma_f32_16x16x32_{f16,bf16}   (D = 128)
//   O^T += V^T P^T   32 x v_mfma_f32_16x16x32_{f16,bf16}
// Every K and V^T operand read from LDS feeds both column blocks.  Computing
// S transposed puts one query per lane column, so the softmax statistics need
// only a 4-lane (xor 16, xor 32) reduction, and the S^T output registers are
// directly the P^T operand of the next product (keys are permuted the same way
// in P^T and in the LDS copy of V^T).
//
// Two ways to finish:
//  * several prefix splits: each split writes its unnormalised state
//    (m, l, acc) to a caller workspace and the tree kernels (tree_attn.hip)
//    merge the splits, walk the ancestors and normalise;
//  * one split (enough query tiles to fill the GPU): the epilogue hands the
//    state to the ancestor walk in the same workgroup (gather_walk4), which
//    normalises and stores O -- no partial state leaves the chip.
#include <algorithm>

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
    float* part_acc;
    int64_t sq_t, sq_h;
    int64_t skp_b, skp_t, skp_h, svp_b, svp_t, svp_h;
    int64_t total_tokens;
    int32_t B, Hq, Hkv, group, max_seqlen, L;
    int32_t n_split, blocks_per_split, qtiles, n_units;
    Divider gdiv;
    float scale_log2;
};

template <typename T, int D, bool FUSED, bool LSE>
__global__ __launch_bounds__(kPrefixThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefix_attn_kernel(
    PrefixParams p, TreeParams tp) {
    constexpr int NC = D / 32;      // MFMA k-chunks over the head dim
    constexpr int ND = D / 16;      // output tiles over the head dim
    // Row strides in elements, padded so a wave's 16-row operand reads hit
    // distinct LDS banks: 288-byte K rows and 160-byte V^T rows read
    // conflict-free on gfx950 (probed; 272- and 144-byte rows did not).
    constexpr int KROW = D + 16;    // Ks row stride in elements
    constexpr int VROW = kBN + 16;  // Vt row stride in elements
    constexpr int DV = D / 8;       // 16-byte vectors per head row
    constexpr int LDS_HALVES = kBN * KROW + D * VROW;
    __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_HALVES];
    uint16_t* Ks = lds;
    uint16_t* Vt = lds + kBN * KROW;

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
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int l16 = lane & 15;
    const int lq = lane >> 4;

    // this lane's query rows (B operand column / output column), one per block
    int64_t qrow[kQB];
    int qh[kQB];
    bool rvalid[kQB];
    Vec16 qf[kQB][NC];
#pragma unroll
    for (int b = 0; b < kQB; ++b) {
        const int rr = qt * kBM + wave * (16 * kQB) + 16 * b + l16;
        rvalid[b] = rr < rows;
        const int tok = rvalid[b] ? divide(rr, p.gdiv) : 0;
        qh[b] = kvh * g + (rr - divide(rr, p.gdiv) * g);
        qrow[b] = (int64_t)s0 + tok;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            qf[b][c] = Vec16{{0u, 0u, 0u, 0u}};
            if (rvalid[b])
                qf[b][c] = ld16((const uint16_t*)p.q + qrow[b] * p.sq_t + (int64_t)qh[b] * p.sq_h + 32 * c + 8 * lq);
        }
    }

    const int k_lo = split * p.blocks_per_split * kBN;
    const int k_hi = (k_lo + p.blocks_per_split * kBN < p.L) ? k_lo + p.blocks_per_split * kBN : p.L;
    const uint16_t* kbase = (const uint16_t*)p.kp + (int64_t)seq * p.skp_b + (int64_t)kvh * p.skp_h;
    const uint16_t* vbase = (const uint16_t*)p.vp + (int64_t)seq * p.svp_b + (int64_t)kvh * p.svp_h;

    float m_run[kQB], l_run[kQB];
    f4_t oacc[kQB][ND];
#pragma unroll
    for (int b = 0; b < kQB; ++b) {
        m_run[b] = -INFINITY;
        l_run[b] = 0.f;
#pragma unroll
        for (int i = 0; i < ND; ++i) oacc[b][i] = f4_t{0.f, 0.f, 0.f, 0.f};
    }

    // ---- K/V block staging, software-pipelined through registers: the loads
    // of block i+1 are issued right after block i is in LDS and land while the
    // MFMAs of block i run ----
    constexpr int KU = kBN * DV / kPrefixThreads;                        // K vectors per thread
    constexpr int VUNITS = (kBN / 4) * DV;                                // 4-key x 8-dim V units
    constexpr int VU = (VUNITS + kPrefixThreads - 1) / kPrefixThreads;   // V units per thread
    static_assert((kBN * DV) % kPrefixThreads == 0 && (VUNITS % 64) == 0, "staging must tile whole waves");
    Vec16 kreg[KU], vreg[VU][4];
    // Keys of the tail block beyond k_hi load row k_hi - 1 instead (always
    // inside the split); their scores are masked to -inf, so P = 0 there.
    auto load_block = [&](int kb) {
#pragma unroll
        for (int i = 0; i < KU; ++i) {
            const int u = tid + i * kPrefixThreads;
            const int key = min(kb + u / DV, k_hi - 1), ch = u % DV;
            kreg[i] = ld16(kbase + (int64_t)key * p.skp_t + 8 * ch);
        }
#pragma unroll
        for (int i = 0; i < VU; ++i) {
            const int u = tid + i * kPrefixThreads;
            const int kg = u % (kBN / 4), dch = u / (kBN / 4);
#pragma unroll
            for (int rk = 0; rk < 4; ++rk) {
                const int key = min(kb + 4 * kg + rk, k_hi - 1);
                if (u < VUNITS) vreg[i][rk] = ld16(vbase + (int64_t)key * p.svp_t + 8 * dch);  // wave-uniform
            }
        }
    };
    auto store_block = [&]() {
#pragma unroll
        for (int i = 0; i < KU; ++i) {
            const int u = tid + i * kPrefixThreads;
            st16(Ks + (u / DV) * KROW + 8 * (u % DV), kreg[i]);
        }
#pragma unroll
        for (int i = 0; i < VU; ++i) {
            const int u = tid + i * kPrefixThreads;
            if (u >= VUNITS) continue;
            const int kg = u % (kBN / 4), dch = u / (kBN / 4);
            const int col = vt_col(4 * kg);
            const Vec16* v4 = vreg[i];
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
    };

    if (k_lo < k_hi) load_block(k_lo);
    // One 64-key block from LDS; MASK instantiates the split's tail block, the
    // only one with keys beyond k_hi, so full blocks carry no masking code.
    auto compute_block = [&](int kb, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        // ---- S^T = K Q^T: lane holds keys 16 mt + 4 lq + i of query l16 ----
        // Software-pipelined: the K operand of step i + 1 is read before the
        // products of step i are issued; step i = (c, mt), consecutive steps
        // accumulate into different key tiles.
        f4_t sacc[kQB][4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int b = 0; b < kQB; ++b) sacc[b][mt] = f4_t{0.f, 0.f, 0.f, 0.f};
        }
        {
            constexpr int NS = 4 * NC;
            Vec16 ka[2];
            ka[0] = ld16(Ks + l16 * KROW + 8 * lq);
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                if (i + 1 < NS) {
                    const int c1 = (i + 1) / 4, mt1 = (i + 1) % 4;
                    ka[(i + 1) & 1] = ld16(Ks + (16 * mt1 + l16) * KROW + 32 * c1 + 8 * lq);
                }
                const int cc = i / 4, mt = i % 4;
#pragma unroll
                for (int b = 0; b < kQB; ++b) sacc[b][mt] = MfmaOps<T>::mma(ka[i & 1], qf[b][cc], sacc[b][mt]);
            }
        }
        // ---- online softmax, per column block.  The running max is kept on
        // raw scores q.k (scale > 0 keeps the order) and the scale*log2(e)
        // factor is folded into the exponent: p = exp2(s c - m c), one FMA ----
        const float c = p.scale_log2;
        if constexpr (MASK) {  // tail block of the split: keys at or beyond k_hi do not exist
#pragma unroll
            for (int b = 0; b < kQB; ++b)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (kb + 16 * mt + 4 * lq + i >= k_hi) sacc[b][mt][i] = -INFINITY;
        }
        // Lazy rescaling: the exponent reference m_run only moves when a block
        // max exceeds it by more than kLazy/c (a factor 2^kLazy in P), so the
        // accumulators are rescaled on a handful of blocks instead of nearly
        // every block.  P stays <= 2^kLazy (exact in fp16/bf16 range, same
        // relative precision) and l carries the same reference, so the final
        // normalisation is unchanged.
        constexpr float kLazy = 8.f;
        Vec16 pf[kQB][2];
        bool rescale = false;
        float alpha[kQB];
#pragma unroll
        for (int b = 0; b < kQB; ++b) {
            float mb = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) mb = fmaxf(mb, sacc[b][mt][i]);
            mb = xor_max(mb, 16);
            mb = xor_max(mb, 32);
            const bool move = (mb - m_run[b]) * c > kLazy;  // always true on the first block
            const float m_new = move ? mb : m_run[b];
            alpha[b] = move ? fast_exp2((m_run[b] - m_new) * c) : 1.f;  // m_run = -inf: 0
            rescale |= move;
            const float mc = m_new * c;
            float psum = 0.f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = fast_exp2(__builtin_fmaf(sacc[b][mt][i], c, -mc));
                    sacc[b][mt][i] = e;
                    psum += e;
                }
            }
            l_run[b] = l_run[b] * alpha[b] + psum;
            m_run[b] = m_new;
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                pf[b][kc].w[0] = MfmaOps<T>::pack2(sacc[b][2 * kc][0], sacc[b][2 * kc][1]);
                pf[b][kc].w[1] = MfmaOps<T>::pack2(sacc[b][2 * kc][2], sacc[b][2 * kc][3]);
                pf[b][kc].w[2] = MfmaOps<T>::pack2(sacc[b][2 * kc + 1][0], sacc[b][2 * kc + 1][1]);
                pf[b][kc].w[3] = MfmaOps<T>::pack2(sacc[b][2 * kc + 1][2], sacc[b][2 * kc + 1][3]);
            }
        }
        // the accumulators need rescaling only when some running max moved
        if (__builtin_expect(__any(rescale), 0)) {
#pragma unroll
            for (int b = 0; b < kQB; ++b) {
#pragma unroll
                for (int dt = 0; dt < ND; ++dt) oacc[b][dt] *= alpha[b];
            }
        }

        // ---- O^T += V^T P^T, two 32-key chunks, pipelined like S: step
        // i = (kc, dt) ----
        {
            constexpr int NS = 2 * ND;
            Vec16 va[2];
            va[0] = ld16(Vt + l16 * VROW + 8 * lq);
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                if (i + 1 < NS) {
                    const int kc1 = (i + 1) / ND, dt1 = (i + 1) % ND;
                    va[(i + 1) & 1] = ld16(Vt + (16 * dt1 + l16) * VROW + 32 * kc1 + 8 * lq);
                }
                const int kc = i / ND, dt = i % ND;
#pragma unroll
                for (int b = 0; b < kQB; ++b) oacc[b][dt] = MfmaOps<T>::mma(va[i & 1], pf[b][kc], oacc[b][dt]);
            }
        }
    };

    // Full blocks in the loop, the split's partial tail block peeled after it,
    // so the loop body is one straight-line copy of compute_block.
    int kb = k_lo;
    for (; kb + kBN <= k_hi; kb += kBN) {
        store_block();
        __syncthreads();
        if (kb + kBN < k_hi) load_block(kb + kBN);
        compute_block(kb, std::false_type{});
        __syncthreads();
    }
    if (kb < k_hi) {
        store_block();
        __syncthreads();
        compute_block(kb, std::true_type{});
        __syncthreads();
    }

    float l_tot[kQB];
#pragma unroll
    for (int b = 0; b < kQB; ++b) {
        l_tot[b] = l_run[b] + __shfl_xor(l_run[b], 16);
        l_tot[b] += __shfl_xor(l_tot[b], 32);
        m_run[b] *= p.scale_log2;  // to the log2 units of the tree walk's scores
    }

    if constexpr (!FUSED) {
        // ---- partial state of this split: (m, l, unnormalised acc) ----
        const int64_t plane = p.total_tokens * (int64_t)p.Hq;
#pragma unroll
        for (int b = 0; b < kQB; ++b) {
            if (!rvalid[b]) continue;
            const int64_t idx = (int64_t)split * plane + qrow[b] * p.Hq + qh[b];
            if (lq == 0) {
                p.part_m[idx] = m_run[b];
                p.part_l[idx] = l_tot[b];
            }
            float* dst = p.part_acc + idx * D + 4 * lq;
#pragma unroll
            for (int dt = 0; dt < ND; ++dt)
                *reinterpret_cast<float4*>(dst + 16 * dt) =
                    make_float4(oacc[b][dt][0], oacc[b][dt][1], oacc[b][dt][2], oacc[b][dt][3]);
        }
    } else {
        // ---- fused epilogue: re-lay each 16-row block in LDS as 4 lanes per
        // query and run the ancestor walk from this state ----
        constexpr int OROW = D + 4;  // fp32 row stride (pad)
        float* Os = reinterpret_cast<float*>(lds) + wave * 16 * OROW;
        float* Ms = reinterpret_cast<float*>(lds) + 4 * 16 * OROW + wave * 32;
        static_assert((4 * 16 * OROW + 4 * 32) * 4 <= LDS_HALVES * 2, "epilogue staging must fit the LDS");
        const int grp = lane >> 2, j = lane & 3;
        constexpr int NCH = D / 32;
#pragma unroll
        for (int b = 0; b < kQB; ++b) {
#pragma unroll
            for (int dt = 0; dt < ND; ++dt)
                *reinterpret_cast<float4*>(Os + l16 * OROW + 16 * dt + 4 * lq) =
                    make_float4(oacc[b][dt][0], oacc[b][dt][1], oacc[b][dt][2], oacc[b][dt][3]);
            if (lq == 0) {
                Ms[l16] = m_run[b];
                Ms[16 + l16] = l_tot[b];
            }
            __syncthreads();
            const int rr = qt * kBM + wave * (16 * kQB) + 16 * b + grp;
            if (rr < rows) {
                const int tok = divide(rr, p.gdiv);
                const int h = kvh * g + (rr - tok * g);
                const int64_t qr = (int64_t)s0 + tok;
                float acc[8 * NCH];
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    const float4 a0 = *reinterpret_cast<const float4*>(Os + grp * OROW + 8 * (j + 4 * i));
                    const float4 a1 = *reinterpret_cast<const float4*>(Os + grp * OROW + 8 * (j + 4 * i) + 4);
                    acc[8 * i + 0] = a0.x;
                    acc[8 * i + 1] = a0.y;
                    acc[8 * i + 2] = a0.z;
                    acc[8 * i + 3] = a0.w;
                    acc[8 * i + 4] = a1.x;
                    acc[8 * i + 5] = a1.y;
                    acc[8 * i + 6] = a1.z;
                    acc[8 * i + 7] = a1.w;
                }
                float m = Ms[grp], l = Ms[16 + grp];
                Vec16 qf4[NCH];
                load_q4<D>(tp, qr, h, j, qf4);
                gather_walk4<T, D, WALK_HEAP, KV_PACKED>(tp, seq, s0, n, tok, kvh, qf4, j, m, l, acc);
                write_out4<T, D, LSE>(tp, qr, h, j, m, l, acc);
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int64_t units_per_split(int batch, int hkv, int max_seqlen, int group) {
    const int64_t qtiles = ((int64_t)max_seqlen * group + kBM - 1) / kBM;
    return (int64_t)batch * hkv * qtiles;
}

// Split count along the prefix: enough work units for ~2 resident workgroups
// on each of 256 CUs, never more splits than 64-key blocks.
static int prefix_splits(int64_t ups, int L, int num_splits, int& blocks_per_split) {
    const int blocks = (L + kBN - 1) / kBN;
    int s = num_splits;
    if (s <= 0) s = (int)std::max<int64_t>(1, (512 + ups / 2) / ups);
    s = std::max(1, std::min(s, std::max(blocks, 1)));
    blocks_per_split = (blocks + s - 1) / s;
    return blocks_per_split > 0 ? (blocks + blocks_per_split - 1) / blocks_per_split : 1;
}

static int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

static int64_t workspace_bytes(int64_t total_tokens, int hq, int head_dim, int splits) {
    if (splits <= 1) return 0;  // one split: fused epilogue, no partial states
    const int64_t plane = total_tokens * hq;
    return 2 * align256(splits * plane * 4) + align256(splits * plane * head_dim * 4);
}

template <typename T, int D>
static int launch_prefix(const PrefixParams& pp, const TreeParams& tp, bool fused, hipStream_t st) {
    const int64_t grid = ((int64_t)pp.n_units + 7) / 8 * 8;
    if (grid >= (int64_t(1) << 31)) {
        set_error("prefix grid too large");
        return QATTN_ERR_ARG;
    }
    if (!fused)
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, false, false>), dim3((unsigned)grid), dim3(kPrefixThreads), 0,
                           st, pp, tp);
    else if (tp.lse)
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, true>), dim3((unsigned)grid), dim3(kPrefixThreads), 0,
                           st, pp, tp);
    else
        hipLaunchKernelGGL((prefix_attn_kernel<T, D, true, false>), dim3((unsigned)grid), dim3(kPrefixThreads), 0,
                           st, pp, tp);
    return launch_status("prefix_attn_kernel");
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
    if (!(scale > 0.f)) {
        set_error("scale must be positive (got %g)", (double)scale);
        return QATTN_ERR_ARG;
    }
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
    const int64_t plane = total_tokens * num_q_heads;
    PrefixParams pp{};
    pp.q = q;
    pp.kp = k_prefix;
    pp.vp = v_prefix;
    pp.cu = cu_seqlens;
    if (!fused) {
        pp.part_m = (float*)workspace;
        pp.part_l = (float*)((char*)workspace + align256(splits * plane * 4));
        pp.part_acc = (float*)((char*)workspace + 2 * align256(splits * plane * 4));
    }
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
        rc = head_dim == 32   ? launch_prefix<F16, 32>(pp, tp, fused, st)
             : head_dim == 64 ? launch_prefix<F16, 64>(pp, tp, fused, st)
                              : launch_prefix<F16, 128>(pp, tp, fused, st);
    } else {
        rc = head_dim == 32   ? launch_prefix<BF16, 32>(pp, tp, fused, st)
             : head_dim == 64 ? launch_prefix<BF16, 64>(pp, tp, fused, st)
                              : launch_prefix<BF16, 128>(pp, tp, fused, st);
    }
    if (rc || fused) return rc;
    tp.part_m = pp.part_m;
    tp.part_l = pp.part_l;
    tp.part_acc = pp.part_acc;
    tp.n_split = splits;
    return run_tree(tp, dtype, head_dim, 0, 0, true, QATTN_ALGO_AUTO, st);
}

}  // extern "C"
