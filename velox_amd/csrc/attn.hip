// Paged attention for verify rows (chain or tree) and prefill, gfx950.
//
// Replaces paged_prefill_attention / paged_decode_attention (reference
// src/paged/metal_kernels.rs MSL :107-191, :307-395; hosts :1227-1383,
// :1680-1846).  The reference walks the KV serially once per (query row,
// q-head); here one wave handles every query row of a sequence tile times
// every q-head of a GQA group against one KV head, so each K/V page is read
// once per (sequence, kv-head, split):
//   * S^T = K . Q^T on v_mfma_f32_16x16x32_{f16,bf16}: K rows come straight
//     from the page (16-byte loads along head_dim), Q^T lives in registers;
//   * online softmax per query column (exp2 with log2e folded into the scale);
//   * O^T = V^T . P^T: P^T is the S^T accumulator re-packed in registers, V is
//     transposed through LDS (key-contiguous rows) so each A fragment is two
//     8-byte LDS reads;
//   * the KV range is split across workgroups (flash-decoding); a second
//     kernel merges the partial (m, l, O) of each (sequence, kv-head, tile) in
//     split order, so results are deterministic and no workgroup waits on
//     another (a device-scope fence costs an XCD-wide L2 writeback on gfx950).
// Visibility: causal (kv_len = kv_offset + t + 1, the reference's rule) or a
// per-row tree mask over the tree slots [kv_offset, kv_offset + 64).
// f32 tensors use a plain per-(row, head) kernel with the reference's loop.
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include <algorithm>
#include <cstdlib>

#include "vx_common.h"

namespace vx {
namespace {

constexpr int kKeyBlock = 64;
constexpr int kAttnWaves = 4;  // waves per workgroup, splitting an item's key blocks
constexpr size_t kAttnCounterBytes = 65536;
constexpr int kMaxQkvSplits = 8;  // split partials the fused qkv finish reads

struct AttnArgs {
    const void *q;
    const void *k;
    const void *v;
    const uint32_t *bt;
    const uint32_t *cu;       // mode 0: cu_seqlens [n_seqs+1]
    const uint32_t *kvo;      // mode 0: kv_offsets; mode 1: kv_lens
    const uint64_t *tmask;    // [total_q] or null
    void *out;
    float *partial;
    int mode;  // 0: varlen rows (cu_seqlens), 1: decode (row i = seq i)
    int n_seqs, n_rows, max_blocks, num_pages, h_q, h_kv, G, D, ps;
    int qr;      // query rows per tile
    int n_qtiles, n_splits, chunk;  // keys per split
    float scale_log2;               // scale * log2(e)
    uint32_t window;
    int out_bf16_round;  // round the output to bf16 before the 16-bit store
    int pnv;             // query vectors per split partial (attn_combine_kernel)
    // Fused qkv finish (mode 0, one query tile per sequence): with qkv set,
    // the query vectors and the sequence's new K/V rows are formed here from
    // the qkv projection's f32 split partials [qkv_splits][total_q][N] --
    // per-head RMSNorm (q_norm / k_norm), RoPE at rope_pos[row], K and V
    // written into the pools at (new_pages[row], new_slots[row]) -- with the
    // arithmetic of qk_rope_scatter_kernel<true>, instead of reading q.
    const float *qkv;
    int qkv_splits;
    const uint16_t *qn_w, *kn_w, *cos_t, *sin_t;  // bf16
    const uint32_t *rope_pos, *new_pages, *new_slots;
    float eps;
};

template <int KT>
struct MfmaT;
template <>
struct MfmaT<VX_F16> {
    typedef half8_t frag;
    static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t cvt(float f) { return f32_to_f16_bits(f); }
};
template <>
struct MfmaT<VX_BF16> {
    typedef bf16x8_t frag;
    static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t cvt(float f) { return f32_to_bf16_bits(f); }
};

__device__ __forceinline__ void row_info(const AttnArgs &a, int seq, int &r_seq, int &row0, int &off) {
    if (a.mode == 0) {
        row0 = (int)a.cu[seq];
        r_seq = (int)a.cu[seq + 1] - row0;
        off = (int)a.kvo[seq];
    } else {
        row0 = seq;
        r_seq = 1;
        off = (int)a.kvo[seq] - 1;  // kv_len - 1 (kv_len 0 handled by the caller)
    }
}

// D: head dim (multiple of 32, <= 256); QT: query tiles of 16 per wave.
// Four waves per workgroup share one item; wave w takes the 64-key blocks
// w, w+4, ... of the item's key range, and the four partial (m, l, O) merge
// through LDS in wave order (deterministic) before the output / split
// partial is written.
template <int KT, int D, int QT>
constexpr size_t attn_lds_bytes() {
    constexpr size_t vt = (size_t)kAttnWaves * D * (kKeyBlock + 4) * 2;
    constexpr size_t comb = (size_t)kAttnWaves * ((D / 16) * QT * 4 + 2 * QT) * 64 * 4;
    return vt > comb ? vt : comb;
}

// FUSE: the instantiation that finishes q/k/v from the qkv partials (a.qkv);
// the plain one compiles without that prologue, whose register arrays would
// otherwise set the register allocation (and occupancy) of every launch.
// The arguments read before the first memory round trip (work item, block
// table, row metadata) also come first as scalars, which the compiler
// preloads into SGPRs at wave launch; they overwrite their copies in `a`.
template <int KT, int D, int QT, bool FUSE>
__global__ __launch_bounds__(256) void paged_attn_kernel(const uint32_t *bt_arg, const uint32_t *cu_arg,
                                                         const uint32_t *kvo_arg, int n_splits_arg, int n_qtiles_arg,
                                                         int h_kv_arg, int max_blocks_arg, int chunk_arg, int ps_arg,
                                                         int mode_arg, AttnArgs a) {
    a.bt = bt_arg;
    a.cu = cu_arg;
    a.kvo = kvo_arg;
    a.n_splits = n_splits_arg;
    a.n_qtiles = n_qtiles_arg;
    a.h_kv = h_kv_arg;
    a.max_blocks = max_blocks_arg;
    a.chunk = chunk_arg;
    a.ps = ps_arg;
    a.mode = mode_arg;
    typedef typename MfmaT<KT>::frag frag;
    constexpr int DK = D / 32;  // MFMA k-steps over head_dim
    constexpr int DT = D / 16;  // output row tiles of O^T
    constexpr int VT_STRIDE = kKeyBlock + 4;  // halves per transposed V row (bank spread)
    // per-wave V^T tiles during the key loop; the merge buffers afterwards
    __shared__ __attribute__((aligned(16))) unsigned char smem[attn_lds_bytes<KT, D, QT>()];

    const int wave = threadIdx.x >> 6;
    uint16_t *vt = (uint16_t *)smem + wave * D * VT_STRIDE;
    const int lane = threadIdx.x & 63;
    const int lq = lane & 15;
    const int lg = lane >> 4;
    int item = blockIdx.x;
    const int split = item % a.n_splits;
    item /= a.n_splits;
    const int qtile = item % a.n_qtiles;
    item /= a.n_qtiles;
    const int hk = item % a.h_kv;
    const int seq = item / a.h_kv;

    // the block-table entry of the wave's first key block depends on neither
    // the row metadata nor the key range: request it with the metadata, so
    // the K/V requests follow one round trip after entry, not two.  The
    // index is clamped to the table row and the page to the pool, so an
    // entry past the sequence's keys is a harmless in-bounds read.
    const uint32_t *btr = a.bt + (int64_t)seq * a.max_blocks;
    uint32_t bt_next = btr[min((split * a.chunk + wave * kKeyBlock + lane) / a.ps, a.max_blocks - 1)];

    int r_seq, row0, off;
    row_info(a, seq, r_seq, row0, off);
    if (a.mode == 1 && (int)a.kvo[seq] == 0) r_seq = 0;  // kv_len 0: zero-filled by the launcher
    const int t0 = qtile * a.qr;
    if (t0 >= r_seq) return;  // empty tile: every split of it exits, no merge needed
    const int t_end = min(r_seq, t0 + a.qr);
    const int nq = max(0, (t_end - t0)) * a.G;  // live query vectors in this tile

    // key range of this tile: causal upper bound or the tree span
    const int kv_end = a.tmask ? off + r_seq : off + t_end;
    const int k_lo = split * a.chunk;
    const int k_hi = min(kv_end, k_lo + a.chunk);

    // ---- fused qkv finish: query vectors into LDS (qbuf[n][D]), this
    // split's new K/V rows into the pools.  One wave per vector; a wave takes
    // its vectors kVB at a time and requests every split partial of the
    // batch before summing, so a batch costs one memory round trip.
    if constexpr (FUSE) {
        constexpr int kVB = 8;
        constexpr int kPairs = (D / 2 + 63) / 64;  // RoPE pairs per lane
        constexpr int kE = 2 * kPairs;             // elements per lane and vector
        uint16_t *qbuf = (uint16_t *)smem;
        for (int i = threadIdx.x; i < (QT * 16 - nq) * D; i += 64 * kAttnWaves) qbuf[nq * D + i] = 0;
        const int t_a = max(0, k_lo - off), t_b = min(r_seq, k_hi - off);
        const int nkv = max(0, t_b - t_a);
        const int nvec = nq + 2 * nkv;
        const int QW = a.h_q * D, KW = a.h_kv * D, N = QW + 2 * KW;
        const int half = D / 2;
        for (int b0 = 0; b0 < nvec; b0 += kAttnWaves * kVB) {
            float pv[kVB][kE][kMaxQkvSplits];
            int kind[kVB], row[kVB], c0[kVB];
            // per-vector metadata and per-lane norm weights / RoPE factors,
            // requested with the partials (not inside the arithmetic below)
            int64_t kv_at[kVB];
            float wn[kVB][kE], cs[kVB][kPairs], sn[kVB][kPairs];
#pragma unroll
            for (int k = 0; k < kVB; k++) {
                const int vi = b0 + wave + kAttnWaves * k;
                kind[k] = vi >= nvec ? 3 : (vi < nq ? 0 : (vi < nq + nkv ? 1 : 2));  // q, k, v, none
                const int t = kind[k] == 0 ? t0 + vi / a.G
                                           : t_a + (kind[k] == 1 ? vi - nq : (kind[k] == 2 ? vi - nq - nkv : 0));
                row[k] = row0 + t;
                c0[k] = kind[k] == 0 ? (hk * a.G + vi % a.G) * D
                                     : (kind[k] == 1 ? QW + hk * D : (kind[k] == 2 ? QW + KW + hk * D : 0));
                const int rr = kind[k] == 3 ? row0 : row[k];
                kv_at[k] = (((int64_t)a.new_pages[rr] * a.h_kv + hk) * a.ps + a.new_slots[rr]) * D;
                const uint32_t pos = a.rope_pos[rr];
                const uint16_t *nw = kind[k] == 0 ? a.qn_w : a.kn_w;
#pragma unroll
                for (int p = 0; p < kPairs; p++) {
                    const int j = min(lane + 64 * p, half - 1);
                    wn[k][p] = bf16_bits_to_f32(nw[j]);
                    wn[k][kPairs + p] = bf16_bits_to_f32(nw[j + half]);
                    cs[k][p] = bf16_bits_to_f32(a.cos_t[(int64_t)pos * half + j]);
                    sn[k][p] = bf16_bits_to_f32(a.sin_t[(int64_t)pos * half + j]);
                }
#pragma unroll
                for (int e = 0; e < kE; e++) {
                    // q/k: element j (e < kPairs) or j + D/2; v: element lane + 64 e
                    const int j = lane + 64 * (e % kPairs);
                    const int c = kind[k] == 2 ? lane + 64 * e : (e < kPairs ? j : j + half);
                    const bool ok = kind[k] < 3 && (kind[k] == 2 ? c < D : j < half);
#pragma unroll
                    for (int sp = 0; sp < kMaxQkvSplits; sp++)
                        pv[k][e][sp] = (ok && sp < a.qkv_splits)
                                           ? a.qkv[((int64_t)sp * a.n_rows + row[k]) * N + c0[k] + c] : 0.f;
                }
            }
#pragma unroll
            for (int k = 0; k < kVB; k++) {
                if (kind[k] == 3) continue;
                float x[kE];
#pragma unroll
                for (int e = 0; e < kE; e++) {
                    float acc = 0.f;
#pragma unroll
                    for (int sp = 0; sp < kMaxQkvSplits; sp++)
                        if (sp < a.qkv_splits) acc += pv[k][e][sp];
                    x[e] = round_to<VX_BF16>(acc);
                }
                if (kind[k] == 2) {
#pragma unroll
                    for (int e = 0; e < kE; e++)
                        if (lane + 64 * e < D) ((uint16_t *)a.v)[kv_at[k] + lane + 64 * e] = MfmaT<KT>::cvt(x[e]);
                    continue;
                }
                float ss = 0.f;
#pragma unroll
                for (int p = 0; p < kPairs; p++) {
                    ss += x[p] * x[p];
                    ss += x[kPairs + p] * x[kPairs + p];
                }
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
                const float m = sqrtf(ss / (float)D + a.eps);
                uint16_t *dst = kind[k] == 0 ? qbuf + (int64_t)(b0 + wave + kAttnWaves * k) * D : (uint16_t *)a.k + kv_at[k];
#pragma unroll
                for (int p = 0; p < kPairs; p++) {
                    const int j = lane + 64 * p;
                    if (j >= half) break;
                    const float av = round_to<VX_BF16>(x[p] / m * wn[k][p]);
                    const float bv = round_to<VX_BF16>(x[kPairs + p] / m * wn[k][kPairs + p]);
                    const float y1 = round_to<VX_BF16>(__fsub_rn(__fmul_rn(av, cs[k][p]), __fmul_rn(bv, sn[k][p])));
                    const float y2 = round_to<VX_BF16>(__fadd_rn(__fmul_rn(av, sn[k][p]), __fmul_rn(bv, cs[k][p])));
                    dst[j] = MfmaT<KT>::cvt(y1);
                    dst[j + half] = MfmaT<KT>::cvt(y2);
                }
            }
        }
        // the new K/V rows and qbuf are read by every wave below
        __syncthreads();
    }

    // ---- Q^T fragments: query n = 16*qt + lq; row t0 + n / G, head hk*G + n % G
    frag qf[QT][DK];
    int q_row[QT];
    uint64_t q_mask[QT];
    int q_lim[QT];
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        const int n = qt * 16 + lq;
        const int t = t0 + n / a.G;
        const bool live = n < nq;
        q_row[qt] = live ? row0 + t : -1;
        q_mask[qt] = (live && a.tmask) ? a.tmask[row0 + t] : 0ull;
        q_lim[qt] = live ? off + t + 1 : 0;  // causal exclusive bound
        const int hq = hk * a.G + (n % a.G);
#pragma unroll
        for (int ks = 0; ks < DK; ks++) {
            uint4 raw = make_uint4(0u, 0u, 0u, 0u);
            if constexpr (FUSE)
                raw = *(const uint4 *)((const uint16_t *)smem + n * D + ks * 32 + lg * 8);
            else if (live)
                raw = *(const uint4 *)((const uint16_t *)a.q + ((int64_t)(row0 + t) * a.h_q + hq) * D + ks * 32 + lg * 8);
            qf[qt][ks] = __builtin_bit_cast(frag, raw);
        }
    }
    // qbuf shares LDS with the V^T tiles of the key loop
    if constexpr (FUSE) __syncthreads();

    floatx4 o[DT][QT];
#pragma unroll
    for (int i = 0; i < DT; i++)
#pragma unroll
        for (int qt = 0; qt < QT; qt++) o[i][qt] = (floatx4){0.f, 0.f, 0.f, 0.f};
    float m_run[QT], l_run[QT];
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        m_run[qt] = -__builtin_inff();
        l_run[qt] = 0.f;
    }

    const int64_t head_stride = (int64_t)a.ps * D;
    const int64_t page_stride = (int64_t)a.h_kv * head_stride;
    const int win = (int)a.window;

    for (int kb = k_lo + wave * kKeyBlock; kb < k_hi; kb += kAttnWaves * kKeyBlock) {
        // ---- request K (4 tiles of 16 keys, lane = key within a tile) and V
        // (lane = key) of the block together, so both round trips overlap.
        // Lane l holds the page of key kb + l (requested one block ahead);
        // the K rows take theirs by lane exchange.
        const int vkey = kb + lane;
        const int vpage = min((int)bt_next, a.num_pages - 1);
        bt_next = btr[min((kb + kAttnWaves * kKeyBlock + lane) / a.ps, a.max_blocks - 1)];
        frag kf[4][DK];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            const int key = kb + mt * 16 + lq;
            const int page = __shfl(vpage, mt * 16 + lq);
            const uint16_t *kr = (const uint16_t *)a.k + page * page_stride + hk * head_stride + (int64_t)(key % a.ps) * D;
#pragma unroll
            for (int ks = 0; ks < DK; ks++) kf[mt][ks] = __builtin_bit_cast(frag, *(const uint4 *)(kr + ks * 32 + lg * 8));
        }
        uint4 vraw[D / 8];
        {
            const uint16_t *vr = (const uint16_t *)a.v + vpage * page_stride + hk * head_stride + (int64_t)(vkey % a.ps) * D;
#pragma unroll
            for (int c = 0; c < D / 8; c++) vraw[c] = *(const uint4 *)(vr + c * 8);
        }
        // keep the V requests ahead of the K . Q^T products: the compiler
        // would otherwise issue them after waiting for K
        __builtin_amdgcn_sched_barrier(0);
        // ---- S^T = K . Q^T
        floatx4 s[4][QT];
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int qt = 0; qt < QT; qt++) {
                floatx4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < DK; ks++) c = MfmaT<KT>::mma(kf[mt][ks], qf[qt][ks], c);
                s[mt][qt] = c;
            }
        // ---- stage V^T for the block: vt[d][key]; the wave's own tile, and
        // LDS operations of one wave complete in order
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int c = 0; c < D / 8; c++) {
            const uint32_t w4[4] = {vraw[c].x, vraw[c].y, vraw[c].z, vraw[c].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                vt[(c * 8 + 2 * e) * VT_STRIDE + lane] = (uint16_t)(w4[e] & 0xffffu);
                vt[(c * 8 + 2 * e + 1) * VT_STRIDE + lane] = (uint16_t)(w4[e] >> 16);
            }
        }
        // ---- mask, scale, block max
        float bmax[QT];
#pragma unroll
        for (int qt = 0; qt < QT; qt++) {
            bmax[qt] = -__builtin_inff();
            // visible keys: [lo, hi) for the causal rule (plus the window); the
            // tree rule also tests the row's ancestor bits past the context
            const int hi = q_row[qt] < 0 ? 0 : min(k_hi, a.tmask ? kv_end : q_lim[qt]);
            const int lo = (win > 0 && q_lim[qt] > win) ? q_lim[qt] - win : 0;
            if (a.tmask) {
#pragma unroll
                for (int mt = 0; mt < 4; mt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int key = kb + mt * 16 + lg * 4 + r;
                        bool vis = key >= lo && key < hi;
                        if (key >= off) vis = vis && (key - off) < 64 && ((q_mask[qt] >> (key - off)) & 1ull);
                        const float v = vis ? s[mt][qt][r] * a.scale_log2 : -__builtin_inff();
                        s[mt][qt][r] = v;
                        bmax[qt] = fmaxf(bmax[qt], v);
                    }
            } else {
#pragma unroll
                for (int mt = 0; mt < 4; mt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int key = kb + mt * 16 + lg * 4 + r;
                        const float v = (key >= lo && key < hi) ? s[mt][qt][r] * a.scale_log2 : -__builtin_inff();
                        s[mt][qt][r] = v;
                        bmax[qt] = fmaxf(bmax[qt], v);
                    }
            }
            bmax[qt] = fmaxf(bmax[qt], __shfl_xor(bmax[qt], 16));
            bmax[qt] = fmaxf(bmax[qt], __shfl_xor(bmax[qt], 32));
        }
        // ---- probabilities, running stats, rescale O
        frag pf[QT][2];
#pragma unroll
        for (int qt = 0; qt < QT; qt++) {
            const float m_new = fmaxf(m_run[qt], bmax[qt]);
            const bool dead = m_new == -__builtin_inff();
            const float alpha = dead ? 1.f : __builtin_amdgcn_exp2f(m_run[qt] - m_new);
            float psum = 0.f;
            uint16_t ph[4][4];
#pragma unroll
            for (int mt = 0; mt < 4; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float p = dead ? 0.f : __builtin_amdgcn_exp2f(s[mt][qt][r] - m_new);
                    psum += p;
                    ph[mt][r] = MfmaT<KT>::cvt(p);
                }
            psum += __shfl_xor(psum, 16);
            psum += __shfl_xor(psum, 32);
            l_run[qt] = l_run[qt] * alpha + psum;
            m_run[qt] = m_new;
#pragma unroll
            for (int i = 0; i < DT; i++) o[i][qt] *= alpha;
#pragma unroll
            for (int st = 0; st < 2; st++) {
                unsigned short tmp[8] __attribute__((aligned(16)));
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    tmp[r] = ph[2 * st][r];
                    tmp[4 + r] = ph[2 * st + 1][r];
                }
                pf[qt][st] = *(frag *)tmp;
            }
        }
        __builtin_amdgcn_wave_barrier();
        // ---- O^T += V^T . P^T ; A element e <-> key 32*st + 4*lg + (e < 4 ? e : 12 + e)
#pragma unroll
        for (int i = 0; i < DT; i++) {
            const uint16_t *vrow = vt + (i * 16 + lq) * VT_STRIDE;
#pragma unroll
            for (int st = 0; st < 2; st++) {
                uint2 lo = *(const uint2 *)(vrow + st * 32 + lg * 4);
                uint2 hi = *(const uint2 *)(vrow + st * 32 + 16 + lg * 4);
                const frag vf = __builtin_bit_cast(frag, make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int qt = 0; qt < QT; qt++) o[i][qt] = MfmaT<KT>::mma(vf, pf[qt][st], o[i][qt]);
            }
        }
    }

    // ---- merge the four waves' partials: every wave publishes (m, l, O) and
    // then finishes the d tiles [TPW*w, TPW*(w+1)) for all of its queries,
    // summing the waves in wave order (deterministic)
    constexpr int TPW = DT >= kAttnWaves ? DT / kAttnWaves : 1;
    __syncthreads();  // every wave is done with its V^T tile
    // 16-byte slots: O tile i of query tile qt of wave w at
    // ((w * QT + qt) * DT + i) * 64 + lane, then (m, l) pairs at
    // (w * QT + qt) * 64 + lane (the same LDS as the four-byte layout)
    floatx4 *comb4 = (floatx4 *)smem;
    float2 *combml = (float2 *)(comb4 + (size_t)kAttnWaves * QT * DT * 64);
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        combml[(wave * QT + qt) * 64 + lane] = make_float2(m_run[qt], l_run[qt]);
#pragma unroll
        for (int i = 0; i < DT; i++) comb4[((wave * QT + qt) * DT + i) * 64 + lane] = o[i][qt];
    }
    __syncthreads();
    const int i_lo = wave * TPW;
    if (i_lo >= DT) return;
    floatx4 om[TPW][QT];
    float mm[QT], lm[QT];
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        float2 mlw[kAttnWaves];
        float fw[kAttnWaves];
        float M = -__builtin_inff();
#pragma unroll
        for (int w = 0; w < kAttnWaves; w++) {
            mlw[w] = combml[(w * QT + qt) * 64 + lane];
            M = fmaxf(M, mlw[w].x);
        }
        const bool dead = M == -__builtin_inff();
        float L = 0.f;
#pragma unroll
        for (int t = 0; t < TPW; t++) om[t][qt] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < kAttnWaves; w++) {
            fw[w] = dead ? 0.f : exp2f(mlw[w].x - M);
            L += mlw[w].y * fw[w];
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                const floatx4 ow = comb4[((w * QT + qt) * DT + i_lo + t) * 64 + lane];
#pragma unroll
                for (int r = 0; r < 4; r++) om[t][qt][r] += ow[r] * fw[w];
            }
        }
        mm[qt] = M;
        lm[qt] = L;
    }

    // ---- single split: write the output; else publish (m, l, O) for the merge
    const int64_t tile_id = ((int64_t)seq * a.h_kv + hk) * a.n_qtiles + qtile;
    if (a.n_splits > 1) {
        // partial layout per (tile, split): m[64], l[64], O[64][D]
        float *pbase = a.partial + (tile_id * a.n_splits + split) * (int64_t)(128 + 64 * D);
#pragma unroll
        for (int qt = 0; qt < QT; qt++) {
            const int n = qt * 16 + lq;
            if (lg == 0 && wave == 0) {
                pbase[n] = mm[qt];
                pbase[64 + n] = lm[qt];
            }
#pragma unroll
            for (int t = 0; t < TPW; t++)
                *(float4 *)(pbase + 128 + (int64_t)n * D + (i_lo + t) * 16 + lg * 4) =
                    make_float4(om[t][qt][0], om[t][qt][1], om[t][qt][2], om[t][qt][3]);
        }
        return;
    }
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        if (q_row[qt] < 0) continue;
        const int n = qt * 16 + lq;
        const int hq = hk * a.G + (n % a.G);
        const float inv = 1.0f / lm[qt];
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            uint16_t h[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float val = om[t][qt][r] * inv;
                if (a.out_bf16_round) val = round_to<VX_BF16>(val);
                h[r] = MfmaT<KT>::cvt(val);
            }
            const int64_t oi = ((int64_t)q_row[qt] * a.h_q + hq) * D + (i_lo + t) * 16 + lg * 4;
            *(uint2 *)((uint16_t *)a.out + oi) = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16),
                                                            (uint32_t)h[2] | ((uint32_t)h[3] << 16));
        }
    }
}

// Workgroup barrier that orders LDS only: __syncthreads() is also a release
// of global memory, i.e. a vmcnt(0) wait, which would drain the key blocks
// requested ahead of it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Shared-KV attention: one workgroup per (sequence, KV head, KV split) holds
// all of the item's query vectors (its rows x G query heads, up to 128).  The
// eight waves stage each 64-key block once in LDS -- K row-major with its
// 16-byte chunks XOR-swizzled by row, V transposed (d-major, keys in pairs
// per 32-bit word) -- and wave w runs query tile w (vectors 16 w .. 16 w + 15)
// over every block of the range, with the S^T / P^T / O^T fragment layouts of
// paged_attn_kernel.  The tiled kernel reads an item's KV range once per
// query tile; a 17-node tree with 4 query heads per KV head has 68 vectors,
// i.e. three 32-vector tiles and three reads.  Blocks b + 1 .. b + PF are
// requested into a PF-slot register ring while block b is computed, and the
// block table one block ahead of that; the launcher instantiates PF = 1
// (deeper rings need one workgroup per CU for their registers and measured
// slower).  Keys past the range are staged as zeros.  Splits publish
// (m, l, O) for attn_combine_kernel with kSharedNV vectors per partial.
constexpr int kSharedWaves = 8;
constexpr int kSharedNV = kSharedWaves * 16;

template <int KT, int D>
constexpr size_t attn_shared_lds_bytes() {
    return 2 * ((size_t)kKeyBlock * D * 2 + (size_t)D * (kKeyBlock + 4) * 2);
}

template <int KT, int D, int PF>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(D <= 128 && PF == 1 ? 4 : 2)))
void paged_attn_shared_kernel(const uint32_t *bt_arg, const uint32_t *cu_arg, const uint32_t *kvo_arg,
                              int n_splits_arg, int h_kv_arg, int max_blocks_arg, int chunk_arg, int ps_arg,
                              AttnArgs a) {
    typedef typename MfmaT<KT>::frag frag;
    constexpr int DK = D / 32;               // MFMA k-steps over head_dim
    constexpr int DT = D / 16;               // output row tiles of O^T
    constexpr int CH = D / 8;                // 16-byte chunks per K/V row
    constexpr int VT_STRIDE = kKeyBlock + 4;  // halves per transposed V row
    constexpr int KBYTES = kKeyBlock * D * 2;
    constexpr int BUFBYTES = KBYTES + D * VT_STRIDE * 2;
    constexpr int NT = 64 * kSharedWaves;          // threads
    constexpr int KC = (kKeyBlock * CH + NT - 1) / NT;  // K chunks per thread and block
    constexpr int VC = (32 * CH + NT - 1) / NT;         // V (key pair, chunk) units per thread and block
    __shared__ __attribute__((aligned(16))) unsigned char smem[attn_shared_lds_bytes<KT, D>()];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lq = lane & 15;
    const int lg = lane >> 4;
    const int split = blockIdx.x % n_splits_arg;
    const int item = blockIdx.x / n_splits_arg;
    const int hk = item % h_kv_arg;
    const int seq = item / h_kv_arg;

    const int row0 = (int)cu_arg[seq];
    const int r_seq = (int)cu_arg[seq + 1] - row0;
    const int off = (int)kvo_arg[seq];
    const int nq = r_seq * a.G;  // live query vectors (<= kSharedNV, checked by the launcher)
    if (nq <= 0) return;         // uniform over the workgroup, before any barrier
    const int kv_end = off + r_seq;
    const int k_lo = split * chunk_arg;
    const int k_hi = min(kv_end, k_lo + chunk_arg);
    const int nb = k_hi > k_lo ? (k_hi - k_lo + kKeyBlock - 1) / kKeyBlock : 0;
    const bool busy = wave * 16 < nq;  // this wave has a query tile

    const uint32_t *btr = bt_arg + (int64_t)seq * max_blocks_arg;
    const int64_t head_stride = (int64_t)ps_arg * D;
    const int64_t page_stride = (int64_t)a.h_kv * head_stride;
    const uint16_t *kbase = (const uint16_t *)a.k + hk * head_stride;
    const uint16_t *vbase = (const uint16_t *)a.v + hk * head_stride;

    // staging units of this thread: K chunk idx = tid + NT j (key idx / CH,
    // chunk idx % CH); V unit idx = tid + NT j (key pair idx / CH, chunk
    // idx % CH).  Both are row-major over the lanes of a wave, so each load
    // instruction reads whole rows.
    auto kkey = [&](int j) { return (tid + NT * j) / CH; };
    auto kchk = [&](int j) { return (tid + NT * j) % CH; };
    auto vpair = [&](int j) { return (tid + NT * j) / CH; };
    auto vchk = [&](int j) { return (tid + NT * j) % CH; };
    auto klive = [&](int j) { return tid + NT * j < kKeyBlock * CH; };
    auto vlive = [&](int j) { return tid + NT * j < 32 * CH; };
    // Addressing (the launcher's precondition): a power-of-two page size, so
    // key / ps and key % ps are shifts, and a pool of fewer than 2^31
    // elements, so element offsets fit 32 bits.
    const int lps = __builtin_ctz((unsigned)ps_arg);
    // Block-table entries are loaded unconditionally (the index is clamped
    // to the table row) and clamped to the pool where they are used: a use
    // next to the load would make the compiler wait for every request in
    // flight, the prefetched key blocks included.
    auto page_of = [&](int key) { return btr[min(key >> lps, max_blocks_arg - 1)]; };
    auto row_at = [&](const uint16_t *base, uint32_t page, int key, int chunk) {
        page = min(page, (uint32_t)(a.num_pages - 1));
        return *(const uint4 *)(base + (page * (uint32_t)page_stride + (uint32_t)((key & (ps_arg - 1)) * D + 8 * chunk)));
    };

    // a PF-slot ring: block b's rows and pages live in slot b % PF
    uint32_t kpg[PF][KC], vpg[PF][VC][2];
    uint4 kr[PF][KC], vr[PF][VC][2];
    auto lookup = [&](int b, auto slot_c) __attribute__((always_inline)) {  // pages of this thread's staging keys of block b
        constexpr int SL = decltype(slot_c)::value;
        const int kb = k_lo + b * kKeyBlock;
#pragma unroll
        for (int j = 0; j < KC; j++) kpg[SL][j] = page_of(kb + kkey(j));
#pragma unroll
        for (int j = 0; j < VC; j++) {
            vpg[SL][j][0] = page_of(kb + 2 * vpair(j));
            vpg[SL][j][1] = page_of(kb + 2 * vpair(j) + 1);
        }
    };
    auto request = [&](int b, auto slot_c) __attribute__((always_inline)) {  // K/V rows of block b into registers (zeros past the range)
        constexpr int SL = decltype(slot_c)::value;
        const int kb = k_lo + b * kKeyBlock;
#pragma unroll
        for (int j = 0; j < KC; j++) {
            const int key = kb + kkey(j);
            kr[SL][j] = make_uint4(0u, 0u, 0u, 0u);
            if (klive(j) && key < k_hi) kr[SL][j] = row_at(kbase, kpg[SL][j], key, kchk(j));
        }
#pragma unroll
        for (int j = 0; j < VC; j++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int key = kb + 2 * vpair(j) + h;
                vr[SL][j][h] = make_uint4(0u, 0u, 0u, 0u);
                if (vlive(j) && key < k_hi) vr[SL][j][h] = row_at(vbase, vpg[SL][j][h], key, vchk(j));
            }
    };
    auto stage = [&](int buf, auto slot_c) __attribute__((always_inline)) {  // registers -> LDS buffer
        constexpr int SL = decltype(slot_c)::value;
        unsigned char *kb_s = smem + buf * BUFBYTES;
        uint16_t *vt = (uint16_t *)(kb_s + KBYTES);
#pragma unroll
        for (int j = 0; j < KC; j++)
            if (klive(j)) {
                const int key = kkey(j);
                *(uint4 *)(kb_s + (key * CH + (kchk(j) ^ (key & (CH - 1)))) * 16) = kr[SL][j];
            }
#pragma unroll
        for (int j = 0; j < VC; j++)
            if (vlive(j)) {
                const uint32_t a0[4] = {vr[SL][j][0].x, vr[SL][j][0].y, vr[SL][j][0].z, vr[SL][j][0].w};
                const uint32_t a1[4] = {vr[SL][j][1].x, vr[SL][j][1].y, vr[SL][j][1].z, vr[SL][j][1].w};
                uint32_t *dst = (uint32_t *)(vt + 8 * vchk(j) * VT_STRIDE + 2 * vpair(j));
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    dst[(2 * e) * (VT_STRIDE / 2)] = (a0[e] & 0xffffu) | (a1[e] << 16);
                    dst[(2 * e + 1) * (VT_STRIDE / 2)] = (a0[e] >> 16) | (a1[e] & 0xffff0000u);
                }
            }
    };

    // ---- this wave's query tile: vector n = 16 wave + lq, row t0 + n / G
    frag qf[DK];
    const int n = wave * 16 + lq;
    const bool qlive = n < nq;
    const int tq = n / a.G;
    const int q_row = qlive ? row0 + tq : -1;
    const uint64_t q_mask = (qlive && a.tmask) ? a.tmask[row0 + tq] : 0ull;
    const int q_lim = qlive ? off + tq + 1 : 0;
    const int hq = hk * a.G + (n % a.G);
#pragma unroll
    for (int ks = 0; ks < DK; ks++) {
        uint4 raw = make_uint4(0u, 0u, 0u, 0u);
        if (qlive) raw = *(const uint4 *)((const uint16_t *)a.q + ((int64_t)q_row * a.h_q + hq) * D + ks * 32 + lg * 8);
        qf[ks] = __builtin_bit_cast(frag, raw);
    }
    const int win = (int)a.window;
    const int hi_q = q_row < 0 ? 0 : min(k_hi, a.tmask ? kv_end : q_lim);
    const int lo_q = (win > 0 && q_lim > win) ? q_lim - win : 0;

    floatx4 o[DT];
#pragma unroll
    for (int i = 0; i < DT; i++) o[i] = (floatx4){0.f, 0.f, 0.f, 0.f};
    float m_run = -__builtin_inff(), l_run = 0.f;

    // block b: its slot is staged into LDS buffer b & 1 (a barrier later every
    // wave is past block b - 1, whose buffer block b + 1 overwrites), then the
    // freed slot takes block b + PF and the next slot's pages block b + PF + 1
    auto compute = [&](int b) __attribute__((always_inline)) {
        const int buf = b & 1;
        const unsigned char *ks_s = smem + buf * BUFBYTES;
        const uint16_t *vt = (const uint16_t *)(ks_s + KBYTES);
        const int kb = k_lo + b * kKeyBlock;
        // ---- S^T = K . Q^T; row mt*16 + lq = (mt*16) | lq, so its swizzle is
        // (lq ^ (mt*16)) & (CH-1) and the tile offset an immediate
        // k-step outer: the four key tiles' products are independent, and
        // one k-step of K fragments is live at a time (register budget of
        // four waves per SIMD)
        floatx4 s[4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) s[mt] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < DK; ks++) {
#pragma unroll
            for (int mt = 0; mt < 4; mt++) {
                const int chunk = ((ks * 4 + lg) ^ lq ^ (mt * 16)) & (CH - 1);
                const uint4 raw = *(const uint4 *)(ks_s + mt * 16 * CH * 16 + lq * CH * 16 + chunk * 16);
                s[mt] = MfmaT<KT>::mma(__builtin_bit_cast(frag, raw), qf[ks], s[mt]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // ---- mask, scale, block max (the rules of paged_attn_kernel).  A
        // block of context keys wholly inside the range, below the first
        // query row and with no window is visible to every query (the
        // workgroup-uniform fast path); otherwise the rules are evaluated
        // per score without branches.
        float bmax = -__builtin_inff();
        if (win == 0 && kb + kKeyBlock <= off && kb + kKeyBlock <= k_hi) {
#pragma unroll
            for (int mt = 0; mt < 4; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    s[mt][r] *= a.scale_log2;
                    bmax = fmaxf(bmax, s[mt][r]);
                }
        } else {
            // tree rule as a word over the block's keys (bit j: key kb + j):
            // context keys before off are visible, tree slot key - off per the
            // row's ancestor bits, keys past the 64 slots not; then shifted so
            // that this lane's element (mt, r) is bit 16 mt + r
            uint64_t tv = ~0ull;
            if (a.tmask) {
                const int dd = kb - off;  // workgroup-uniform
                if (dd >= 64)
                    tv = 0ull;
                else if (dd >= 0)
                    tv = q_mask >> dd;
                else if (dd > -64)
                    tv = (q_mask << (-dd)) | ((1ull << (-dd)) - 1ull);
                tv >>= lg * 4;
            }
            const uint32_t tlo = (uint32_t)tv, thi = (uint32_t)(tv >> 32);
#pragma unroll
            for (int mt = 0; mt < 4; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = kb + mt * 16 + lg * 4 + r;
                    const uint32_t bit = ((mt < 2 ? tlo : thi) >> ((mt & 1) * 16 + r)) & 1u;
                    const bool vis = (key >= lo_q) & (key < hi_q) & (bit != 0u);
                    const float v = vis ? s[mt][r] * a.scale_log2 : -__builtin_inff();
                    s[mt][r] = v;
                    bmax = fmaxf(bmax, v);
                }
        }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        // ---- probabilities, running stats, rescale O
        const float m_new = fmaxf(m_run, bmax);
        const bool dead = m_new == -__builtin_inff();
        const float alpha = dead ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
        float psum = 0.f;
        uint16_t ph[4][4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = dead ? 0.f : __builtin_amdgcn_exp2f(s[mt][r] - m_new);
                psum += p;
                ph[mt][r] = MfmaT<KT>::cvt(p);
            }
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // a running max moved
#pragma unroll
            for (int i = 0; i < DT; i++) o[i] *= alpha;
        }
        frag pf[2];
#pragma unroll
        for (int st = 0; st < 2; st++) {
            unsigned short tmp[8] __attribute__((aligned(16)));
#pragma unroll
            for (int r = 0; r < 4; r++) {
                tmp[r] = ph[2 * st][r];
                tmp[4 + r] = ph[2 * st + 1][r];
            }
            pf[st] = *(frag *)tmp;
        }
        // ---- O^T += V^T . P^T ; A element e <-> key 32*st + 4*lg + (e < 4 ? e : 12 + e)
        // key half outer: the d tiles' products are independent; four V^T
        // fragments in flight at a time
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
            for (int i = 0; i < DT; i++) {
                const uint16_t *vrow = vt + (i * 16 + lq) * VT_STRIDE;
                const uint2 lo = *(const uint2 *)(vrow + st * 32 + lg * 4);
                const uint2 hi = *(const uint2 *)(vrow + st * 32 + 16 + lg * 4);
                const frag vf = __builtin_bit_cast(frag, make_uint4(lo.x, lo.y, hi.x, hi.y));
                o[i] = MfmaT<KT>::mma(vf, pf[st], o[i]);
                if (i % 4 == 3) __builtin_amdgcn_sched_barrier(0);
            }
        };
    auto iter = [&](int b, auto slot_c) __attribute__((always_inline)) {
        constexpr int SL = decltype(slot_c)::value;
        stage(b & 1, slot_c);
        lds_barrier();
        if (b + PF < nb) request(b + PF, slot_c);
        if (b + PF + 1 < nb) lookup(b + PF + 1, std::integral_constant<int, (SL + 1) % PF>{});
        if (busy) compute(b);
    };
    lookup(0, std::integral_constant<int, 0>{});
    if constexpr (PF > 1) if (1 < nb) lookup(1, std::integral_constant<int, 1 % PF>{});
    if constexpr (PF > 2) if (2 < nb) lookup(2, std::integral_constant<int, 2 % PF>{});
    if (0 < nb) request(0, std::integral_constant<int, 0>{});
    if constexpr (PF > 1) if (1 < nb) request(1, std::integral_constant<int, 1 % PF>{});
    if constexpr (PF > 2) if (2 < nb) request(2, std::integral_constant<int, 2 % PF>{});
    if (PF < nb) lookup(PF, std::integral_constant<int, 0>{});
    int b = 0;
    for (; b + PF <= nb; b += PF) {
        iter(b, std::integral_constant<int, 0>{});
        if constexpr (PF > 1) iter(b + 1, std::integral_constant<int, 1 % PF>{});
        if constexpr (PF > 2) iter(b + 2, std::integral_constant<int, 2 % PF>{});
    }
    if (b < nb) iter(b, std::integral_constant<int, 0>{});
    if constexpr (PF > 2) if (b + 1 < nb) iter(b + 1, std::integral_constant<int, 1 % PF>{});
    if (!busy) return;

    if (!qlive) return;  // the merge reads live vectors only
    const int64_t item_id = (int64_t)seq * a.h_kv + hk;
    if (n_splits_arg > 1) {
        // partial layout per (item, split): m[NV], l[NV], O[NV][D]
        float *pbase = a.partial + (item_id * n_splits_arg + split) * (int64_t)(2 * kSharedNV + kSharedNV * D);
        if (lg == 0) {
            pbase[n] = m_run;
            pbase[kSharedNV + n] = l_run;
        }
#pragma unroll
        for (int i = 0; i < DT; i++)
            *(float4 *)(pbase + 2 * kSharedNV + (int64_t)n * D + i * 16 + lg * 4) =
                make_float4(o[i][0], o[i][1], o[i][2], o[i][3]);
        return;
    }
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int i = 0; i < DT; i++) {
        uint16_t h[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float val = o[i][r] * inv;
            if (a.out_bf16_round) val = round_to<VX_BF16>(val);
            h[r] = MfmaT<KT>::cvt(val);
        }
        const int64_t oi = ((int64_t)q_row * a.h_q + hq) * D + i * 16 + lg * 4;
        *(uint2 *)((uint16_t *)a.out + oi) = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16),
                                                        (uint32_t)h[2] | ((uint32_t)h[3] << 16));
    }
}

// Merge the split partials of each (sequence, kv-head, tile) in split order;
// a partial holds a.pnv vectors: m[pnv], l[pnv], O[pnv][D].  One thread per
// (tile, vector, four consecutive d), nv vectors per tile; the splits'
// statistics and values are requested eight splits at a time, so a merge of
// up to eight splits costs one memory round trip.
template <int KT>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a, int nv) {
    constexpr int kB = 8;
    const int D4 = a.D / 4;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_tile = (int64_t)nv * D4;
    int64_t item = gid / per_tile;
    const int rem = (int)(gid - item * per_tile);
    const int n = rem / D4;
    const int d = (rem - n * D4) * 4;
    const int qtile = (int)(item % a.n_qtiles);
    item /= a.n_qtiles;
    const int hk = (int)(item % a.h_kv);
    const int seq = (int)(item / a.h_kv);
    if (seq >= a.n_seqs) return;
    int r_seq, row0, off;
    row_info(a, seq, r_seq, row0, off);
    if (a.mode == 1 && (int)a.kvo[seq] == 0) r_seq = 0;
    const int t0 = qtile * a.qr;
    if (t0 >= r_seq) return;
    const int nq = (min(r_seq, t0 + a.qr) - t0) * a.G;
    if (n >= nq) return;
    const int64_t tile_id = ((int64_t)seq * a.h_kv + hk) * a.n_qtiles + qtile;
    const int64_t stride = (int64_t)a.pnv * (2 + a.D);
    const float *p0 = a.partial + tile_id * a.n_splits * stride;
    float L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    auto load_batch = [&](int s0, float (&mb)[kB], float (&lb)[kB], float4 (&ob)[kB]) {
#pragma unroll
        for (int j = 0; j < kB; j++) {
            const bool ok = s0 + j < a.n_splits;
            const float *ps = p0 + (int64_t)(s0 + j) * stride;
            mb[j] = ok ? ps[n] : -__builtin_inff();
            lb[j] = ok ? ps[a.pnv + n] : 0.f;
            ob[j] = ok ? *(const float4 *)(ps + 2 * a.pnv + (int64_t)n * a.D + d) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto add_batch = [&](int s0, float M, const float (&mb)[kB], const float (&lb)[kB], const float4 (&ob)[kB]) {
#pragma unroll
        for (int j = 0; j < kB; j++) {
            if (s0 + j >= a.n_splits) break;
            const float f = mb[j] == -__builtin_inff() ? 0.f : exp2f(mb[j] - M);
            L += lb[j] * f;
            acc.x += ob[j].x * f;
            acc.y += ob[j].y * f;
            acc.z += ob[j].z * f;
            acc.w += ob[j].w * f;
        }
    };
    if (a.n_splits <= kB) {
        // one batch: the maximum comes from the loaded statistics
        float mb[kB], lb[kB];
        float4 ob[kB];
        load_batch(0, mb, lb, ob);
        float M = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < kB; j++) M = fmaxf(M, mb[j]);
        add_batch(0, M, mb, lb, ob);
    } else {
        // the maximum first, then the sum in split order, eight splits a batch
        float M = -__builtin_inff();
        for (int s0 = 0; s0 < a.n_splits; s0 += kB) {
            float mb[kB];
#pragma unroll
            for (int j = 0; j < kB; j++) mb[j] = s0 + j < a.n_splits ? p0[(s0 + j) * stride + n] : -__builtin_inff();
#pragma unroll
            for (int j = 0; j < kB; j++) M = fmaxf(M, mb[j]);
        }
        for (int s0 = 0; s0 < a.n_splits; s0 += kB) {
            float mb[kB], lb[kB];
            float4 ob[kB];
            load_batch(s0, mb, lb, ob);
            add_batch(s0, M, mb, lb, ob);
        }
    }
    const float vals[4] = {acc.x / L, acc.y / L, acc.z / L, acc.w / L};
    uint16_t h[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float val = vals[r];
        if (a.out_bf16_round) val = round_to<VX_BF16>(val);
        h[r] = MfmaT<KT>::cvt(val);
    }
    const int t = t0 + n / a.G;
    const int hq = hk * a.G + (n % a.G);
    *(uint2 *)((uint16_t *)a.out + ((int64_t)(row0 + t) * a.h_q + hq) * a.D + d) =
        make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
}

void launch_combine(const AttnArgs &a, int dtype, int64_t n_tiles, int nv, hipStream_t st) {
    const unsigned grid = (unsigned)vx_cdiv(n_tiles * nv * (a.D / 4), 256);
    if (dtype == VX_F16)
        hipLaunchKernelGGL(attn_combine_kernel<VX_F16>, dim3(grid), dim3(256), 0, st, a, nv);
    else
        hipLaunchKernelGGL(attn_combine_kernel<VX_BF16>, dim3(grid), dim3(256), 0, st, a, nv);
}

// Plain per-(row, q-head) kernel, the reference's loop (MSL :307-395 / :107-191)
// with a fixed-order tree reduction of q.k; used for f32 tensors.
template <int DT>
__global__ void paged_attn_ref_kernel(AttnArgs a, int64_t total_q) {
    extern __shared__ float sh[];
    float *qs = sh;
    float *red = sh + a.D;
    const int row = blockIdx.x;
    const int hq = blockIdx.y;
    const int tid = threadIdx.x;
    int seq = 0;
    if (a.mode == 0) {
        int lo = 0, hi = a.n_seqs - 1;
        while (lo < hi) {  // last seq with cu[seq] <= row
            const int mid = (lo + hi + 1) / 2;
            if ((int)a.cu[mid] <= row) lo = mid; else hi = mid - 1;
        }
        seq = lo;
    } else {
        seq = row;
    }
    int r_seq, row0, off;
    row_info(a, seq, r_seq, row0, off);
    const int t = row - row0;
    const int hk = hq / a.G;
    int end = a.tmask ? off + r_seq : off + t + 1;
    if (a.mode == 1) end = (int)a.kvo[seq];
    const int self_len = off + t + 1;
    const int start = (a.window > 0 && self_len > (int)a.window) ? self_len - (int)a.window : 0;
    if (tid < a.D) qs[tid] = ld_elem<DT>(a.q, ((int64_t)row * a.h_q + hq) * a.D + tid);
    __syncthreads();
    float acc = 0.f, m = -__builtin_inff(), l = 0.f;
    const uint64_t tm = a.tmask ? a.tmask[row] : 0ull;
    for (int pos = start; pos < end; pos++) {
        if (a.tmask && pos >= off) {
            const int j = pos - off;
            if (j >= 64 || !((tm >> j) & 1ull)) continue;
        }
        const int page = min((int)a.bt[(int64_t)seq * a.max_blocks + min(pos / a.ps, a.max_blocks - 1)], a.num_pages - 1);
        const int64_t base = (((int64_t)page * a.h_kv + hk) * a.ps + pos % a.ps) * a.D;
        red[tid] = tid < a.D ? qs[tid] * ld_elem<DT>(a.k, base + tid) : 0.f;
        __syncthreads();
        for (int stride = blockDim.x / 2; stride > 0; stride >>= 1) {
            if (tid < stride) red[tid] += red[tid + stride];
            __syncthreads();
        }
        const float s = red[0] * (a.scale_log2 * 0.69314718055994531f);
        __syncthreads();
        const float new_m = fmaxf(m, s);
        const float alpha = __expf(m - new_m);
        const float beta = __expf(s - new_m);
        if (tid < a.D) acc = acc * alpha + beta * ld_elem<DT>(a.v, base + tid);
        l = l * alpha + beta;
        m = new_m;
    }
    if (tid < a.D) st_elem<DT>(a.out, ((int64_t)row * a.h_q + hq) * a.D + tid, l > 0.f ? acc / l : 0.f);
}

__global__ void zero_u16_kernel(uint16_t *p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

template <int KT, int D, int QT>
void launch_attn(const AttnArgs &a, int64_t n_items, hipStream_t st) {
    if (a.qkv)
        hipLaunchKernelGGL((paged_attn_kernel<KT, D, QT, true>), dim3((unsigned)n_items), dim3(64 * kAttnWaves), 0,
                           st, a.bt, a.cu, a.kvo, a.n_splits, a.n_qtiles, a.h_kv, a.max_blocks, a.chunk, a.ps, a.mode,
                           a);
    else
        hipLaunchKernelGGL((paged_attn_kernel<KT, D, QT, false>), dim3((unsigned)n_items), dim3(64 * kAttnWaves), 0,
                           st, a.bt, a.cu, a.kvo, a.n_splits, a.n_qtiles, a.h_kv, a.max_blocks, a.chunk, a.ps, a.mode,
                           a);
}

template <int KT>
int dispatch_attn(const AttnArgs &a, int QT, int64_t n_items, hipStream_t st) {
#define VX_ACASE(d, qt)                                       \
    if (a.D == d && QT == qt) {                              \
        launch_attn<KT, d, qt>(a, n_items, st);              \
        return 0;                                            \
    }
    VX_ACASE(32, 1) VX_ACASE(32, 2) VX_ACASE(32, 4)
    VX_ACASE(64, 1) VX_ACASE(64, 2) VX_ACASE(64, 4)
    VX_ACASE(128, 1) VX_ACASE(128, 2) VX_ACASE(128, 4)
    VX_ACASE(256, 1) VX_ACASE(256, 2)
#undef VX_ACASE
    return set_error("paged_attention: no kernel for head_dim");
}

template <int KT>
int dispatch_attn_shared(const AttnArgs &a, int pf, int64_t n_items, hipStream_t st) {
#define VX_SCASE(d, p)                                                                                     \
    if (a.D == d && pf == p) {                                                                             \
        hipLaunchKernelGGL((paged_attn_shared_kernel<KT, d, p>), dim3((unsigned)n_items),                  \
                           dim3(64 * kSharedWaves), 0, st, a.bt, a.cu, a.kvo, a.n_splits, a.h_kv,          \
                           a.max_blocks, a.chunk, a.ps, a);                                                \
        return 0;                                                                                          \
    }
    VX_SCASE(32, 1) VX_SCASE(64, 1) VX_SCASE(128, 1) VX_SCASE(256, 1)
#undef VX_SCASE
    return set_error("paged_attention: no kernel for head_dim");
}

// The shared-KV kernel takes a sequence's query vectors when they exceed one
// 32-vector tile and fit its eight waves (mode 0, 16-bit, no fused qkv
// finish), for power-of-two page sizes and pools of fewer than 2^31 elements;
// VX_ATTN_SHARED=0 turns it off.
bool use_shared_attn(int mode, int64_t max_rows, int64_t G, int64_t D, int64_t ps, int64_t pool_elems) {
    const char *env = getenv("VX_ATTN_SHARED");
    if (env && env[0] == '0') return false;
    const int64_t v = max_rows * G;
    return mode == 0 && v > 32 && v <= kSharedNV && (D == 32 || D == 64 || D == 128 || D == 256) && ps > 0 &&
           (ps & (ps - 1)) == 0 && pool_elems < (1ll << 31);
}

// Its prefetch depth: one key block in flight in registers, two workgroups
// per CU (D <= 128).  Deeper rings (two or three blocks, one workgroup per
// CU for the registers) measured slower on config 3's tree step.
int shared_attn_depth(int64_t) { return 1; }

// Its KV split: ~2 workgroups per CU at depth 1 with D <= 128 (one otherwise:
// the registers or, at D = 256, the LDS fill a CU), at least two key blocks
// per split.  VX_ATTN_SHARED_SPLITS overrides the count.
void shared_attn_plan(int64_t base_items, int64_t max_kv, int64_t D, int pf, int64_t &splits, int64_t &chunk) {
    const int64_t max_keys = std::max<int64_t>(1, max_kv);
    const int64_t per_cu = D <= 128 && pf == 1 ? 2 : 1;
    splits = std::max<int64_t>(1, per_cu * device_cu_count() / std::max<int64_t>(1, base_items));
    const char *env = getenv("VX_ATTN_SHARED_SPLITS");
    if (env && *env) splits = std::max(1, atoi(env));
    chunk = vx_cdiv(vx_cdiv(max_keys, splits), kKeyBlock) * kKeyBlock;
    chunk = std::max<int64_t>(chunk, 2 * kKeyBlock);
    splits = vx_cdiv(max_keys, chunk);
}

}  // namespace

size_t attn_workspace_bytes(int64_t n_seqs, int64_t h_kv, int64_t n_qtiles, int64_t n_splits, int64_t D) {
    if (n_splits <= 1) return kAttnCounterBytes;
    return kAttnCounterBytes + (size_t)n_seqs * h_kv * n_qtiles * n_splits * (128 + 64 * D) * 4;
}

// Upper bound of the workspace paged_attention_launch needs for any batch
// within these limits (either kernel, splits of at least 128 keys).
size_t attn_workspace_bound(int64_t n_seqs, int64_t h_kv, int64_t max_rows, int64_t G, int64_t D, int64_t max_kv) {
    const int64_t qn_max = D <= 128 ? 64 : 32;
    int64_t qt = std::max<int64_t>(1, vx_cdiv(std::min<int64_t>(max_rows * G, qn_max), 16));
    if (qt == 3) qt = 4;
    const int64_t qr = std::max<int64_t>(1, qt * 16 / G);
    const int64_t nqt = vx_cdiv(max_rows, qr);
    const int64_t splits = std::max<int64_t>(1, vx_cdiv(max_kv, 2 * kKeyBlock));
    size_t need = attn_workspace_bytes(n_seqs, h_kv, nqt, splits, D);
    if (use_shared_attn(0, max_rows, G, D, 1, 0) && splits > 1)
        need = std::max(need, kAttnCounterBytes + (size_t)n_seqs * h_kv * splits * kSharedNV * (2 + D) * 4);
    return need;
}

// Shared launcher for the C ABI and the engine.
int paged_attention_launch(const void *q, const void *k_pool, const void *v_pool, const uint32_t *bt,
                           const uint32_t *cu, const uint32_t *kvo, const uint64_t *tmask, void *out,
                           int mode, int64_t total_q, int64_t n_seqs, int64_t max_rows,
                           int64_t max_blocks, int64_t num_pages, int64_t h_q, int64_t h_kv,
                           int64_t D, int64_t ps, float scale, uint32_t window, int dtype,
                           void *workspace, size_t ws_bytes, int64_t max_kv, hipStream_t st,
                           int out_bf16_round, const AttnQkvFuse *fuse) {
    AttnArgs a{};
    a.out_bf16_round = out_bf16_round;
    a.n_rows = (int)total_q;
    if (fuse) {
        a.qkv = fuse->partial;
        a.qkv_splits = fuse->splits;
        a.qn_w = fuse->qn;
        a.kn_w = fuse->kn;
        a.cos_t = fuse->cos_t;
        a.sin_t = fuse->sin_t;
        a.rope_pos = fuse->pos;
        a.new_pages = fuse->pages;
        a.new_slots = fuse->slots;
        a.eps = fuse->eps;
    }
    a.q = q;
    a.k = k_pool;
    a.v = v_pool;
    a.bt = bt;
    a.cu = cu;
    a.kvo = kvo;
    a.tmask = tmask;
    a.out = out;
    a.mode = mode;
    a.n_seqs = (int)n_seqs;
    a.max_blocks = (int)max_blocks;
    a.num_pages = (int)num_pages;
    a.h_q = (int)h_q;
    a.h_kv = (int)h_kv;
    a.G = (int)(h_q / h_kv);
    a.D = (int)D;
    a.ps = (int)ps;
    a.scale_log2 = scale * 1.44269504088896341f;
    a.window = window;
    if (total_q == 0 || n_seqs == 0) return 0;
    // the kernels read the block table before they know the key range
    if (max_blocks < 1 || num_pages < 1 || ps < 1) return set_error("paged_attention: empty pool or block table");
    if (dtype == VX_F32) {
        const int threads = 256;
        hipLaunchKernelGGL(paged_attn_ref_kernel<VX_F32>, dim3((unsigned)total_q, (unsigned)h_q), dim3(threads),
                           (size_t)(D + threads) * 4, st, a, total_q);
        VX_HIP(hipGetLastError());
        return 0;
    }
    a.pnv = 64;
    if (use_shared_attn(mode, max_rows, a.G, D, ps, num_pages * h_kv * ps * D) && !fuse) {
        // one workgroup per (sequence, KV head, split) over all query vectors
        const int64_t base_items = n_seqs * h_kv;
        int64_t splits, chunk;
        const int pf = shared_attn_depth(D);
        shared_attn_plan(base_items, max_kv, D, pf, splits, chunk);
        a.n_qtiles = 1;
        a.qr = (int)max_rows;
        a.pnv = kSharedNV;
        a.chunk = (int)chunk;
        a.n_splits = (int)splits;
        void *ws = workspace;
        const size_t need = kAttnCounterBytes + (size_t)base_items * splits * kSharedNV * (2 + D) * 4;
        if (splits > 1) {
            if (!ws) {
                VX_TRY(stream_workspace(st, need, &ws));
            } else if (ws_bytes < need) {
                return set_error("paged_attention: workspace too small");
            }
        }
        a.partial = ws ? (float *)((char *)ws + kAttnCounterBytes) : nullptr;
        const int64_t n_items = base_items * splits;
        int rc = dtype == VX_F16 ? dispatch_attn_shared<VX_F16>(a, pf, n_items, st)
                                 : dispatch_attn_shared<VX_BF16>(a, pf, n_items, st);
        if (rc) return rc;
        if (splits > 1) launch_combine(a, dtype, base_items, (int)std::min<int64_t>(kSharedNV, max_rows * a.G), st);
        VX_HIP(hipGetLastError());
        return 0;
    }
    // Query vectors per tile.  Every query tile reads the sequence's whole KV
    // range, and the 64-vector tile is a heavy kernel (one workgroup per CU).
    // When a sequence's queries need two 64-vector tiles anyway (65..128, e.g.
    // a 17-node tree times 4 query heads per KV head), 32-vector tiles are
    // faster: 11.3 vs 21.6 ms per tree-verify step of 16 x 17 rows at context
    // 2048.  Long prefill keeps the 64-vector tile (5 % faster there).
    // VX_ATTN_QN overrides the cap.
    const char *qn_env = getenv("VX_ATTN_QN");
    int qn_max = D <= 128 ? 64 : 32;
    if (qn_max == 64 && max_rows * a.G > 64 && max_rows * a.G <= 128) qn_max = 32;
    if (qn_env && *qn_env) qn_max = atoi(qn_env);
    int64_t qn = std::min<int64_t>(max_rows * a.G, qn_max);
    int QT = (int)std::max<int64_t>(1, vx_cdiv(qn, 16));
    if (QT == 3) QT = 4;
    a.qr = std::max(1, (QT * 16) / a.G);
    a.n_qtiles = (int)vx_cdiv(max_rows, a.qr);
    if (fuse && (mode != 0 || a.n_qtiles != 1 || dtype == VX_F32 || fuse->splits < 1 || fuse->splits > kMaxQkvSplits))
        return set_error("paged_attention: the fused qkv finish needs one query tile per sequence (mode 0, 16-bit) "
                         "and at most 8 qkv splits");
    // KV split across workgroups (each workgroup's four waves already split
    // its range): aim for ~2 workgroups per CU, at least one key block per wave
    const int64_t base_items = n_seqs * h_kv * a.n_qtiles;
    const int64_t max_keys = std::max<int64_t>(1, max_kv);
    const int64_t target = 2LL * device_cu_count();
    int64_t splits = std::max<int64_t>(1, target / std::max<int64_t>(1, base_items));
    int64_t chunk = vx_cdiv(vx_cdiv(max_keys, splits), kKeyBlock) * kKeyBlock;
    chunk = std::max<int64_t>(chunk, kAttnWaves * kKeyBlock);
    splits = vx_cdiv(max_keys, chunk);
    a.chunk = (int)chunk;
    a.n_splits = (int)splits;
    void *ws = workspace;
    const size_t need = attn_workspace_bytes(n_seqs, h_kv, a.n_qtiles, splits, D);
    if (splits > 1) {
        if (!ws) {
            VX_TRY(stream_workspace(st, need, &ws));
        } else if (ws_bytes < need) {
            return set_error("paged_attention: workspace too small");
        }
    }
    a.partial = ws ? (float *)((char *)ws + kAttnCounterBytes) : nullptr;
    if (mode == 1) {
        // decode rows with kv_len == 0 keep zeros (metal_kernels.rs:2395-2397)
        const int64_t tot = total_q * h_q * D;
        hipLaunchKernelGGL(zero_u16_kernel, dim3((unsigned)vx_cdiv(tot, 256)), dim3(256), 0, st, (uint16_t *)out, tot);
    }
    const int64_t n_items = base_items * splits;
    int rc = dtype == VX_F16 ? dispatch_attn<VX_F16>(a, QT, n_items, st) : dispatch_attn<VX_BF16>(a, QT, n_items, st);
    if (rc) return rc;
    if (splits > 1) launch_combine(a, dtype, base_items, std::min(64, a.qr * a.G), st);
    VX_HIP(hipGetLastError());
    return 0;
}

}  // namespace vx

using namespace vx;

static int check_attn_shapes(int64_t h_q, int64_t h_kv, int64_t D, int dtype) {
    VX_REQUIRE(h_kv > 0 && h_q % h_kv == 0, "paged_attention: H_q must be divisible by H_kv");
    VX_REQUIRE(D <= 256, "paged_attention: head_dim > D_MAX 256");
    VX_REQUIRE(D % 32 == 0, "paged_attention: head_dim must be a multiple of 32");
    VX_REQUIRE(dtype == VX_F32 || dtype == VX_F16 || dtype == VX_BF16, "paged_attention: unsupported dtype");
    return 0;
}

extern "C" int vx_paged_attention(const void *q, const void *k_pool, const void *v_pool,
                                  const uint32_t *block_table, const uint32_t *cu_seqlens,
                                  const uint32_t *seq_id_per_q, const uint32_t *kv_offsets,
                                  const uint64_t *tree_mask, void *out, int64_t total_q,
                                  int64_t n_seqs, int64_t max_blocks, int64_t num_pages,
                                  int64_t h_q, int64_t h_kv, int64_t head_dim, int64_t page_size,
                                  float scale, uint32_t sliding_window, int dtype, void *stream) {
    VX_TRY(check_attn_shapes(h_q, h_kv, head_dim, dtype));
    if (total_q == 0 || n_seqs == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(q && k_pool && v_pool && block_table && cu_seqlens && kv_offsets && out,
               "paged_attention: null tensor");
    VX_REQUIRE(max_blocks > 0 && num_pages > 0 && page_size > 0, "paged_attention: empty pool");
    VX_REQUIRE(seq_id_per_q, "paged_attention: null tensor");
    // The reference's kernel finds a row's sequence through seq_id_per_q and
    // its position through cu_seqlens (MSL :307-395); this kernel walks the
    // cu_seqlens ranges, so the two must describe the same rows.  They are
    // checked on the host (one small copy and a stream synchronisation), which
    // also gives the launch plan the longest row range and key range.
    int64_t max_rows = 1, max_kv = 1;
    {
        hipStream_t st = (hipStream_t)stream;
        std::vector<uint32_t> cu((size_t)n_seqs + 1), sid((size_t)total_q), kvo((size_t)n_seqs);
        VX_HIP(hipMemcpyAsync(cu.data(), cu_seqlens, cu.size() * 4, hipMemcpyDeviceToHost, st));
        VX_HIP(hipMemcpyAsync(sid.data(), seq_id_per_q, sid.size() * 4, hipMemcpyDeviceToHost, st));
        VX_HIP(hipMemcpyAsync(kvo.data(), kv_offsets, kvo.size() * 4, hipMemcpyDeviceToHost, st));
        VX_HIP(hipStreamSynchronize(st));
        VX_REQUIRE(cu[0] == 0 && (int64_t)cu[n_seqs] == total_q, "paged_attention: cu_seqlens must run from 0 to total_q");
        for (int64_t s = 0; s < n_seqs; s++)
            VX_REQUIRE(cu[s] <= cu[s + 1], "paged_attention: cu_seqlens must be non-decreasing");
        for (int64_t row = 0; row < total_q; row++) {
            const uint32_t sq = sid[row];
            VX_REQUIRE(sq < (uint64_t)n_seqs && cu[sq] <= (uint64_t)row && (uint64_t)row < cu[sq + 1],
                       "paged_attention: seq_id_per_q[" + std::to_string(row) + "] disagrees with cu_seqlens");
        }
        for (int64_t s = 0; s < n_seqs; s++) {
            const int64_t r = (int64_t)cu[s + 1] - cu[s];
            max_rows = std::max(max_rows, r);
            max_kv = std::max(max_kv, (int64_t)kvo[s] + r);
        }
        max_kv = std::min(max_kv, max_blocks * page_size);  // the block table bounds the key range
    }
    return paged_attention_launch(q, k_pool, v_pool, block_table, cu_seqlens, kv_offsets, tree_mask,
                                  out, 0, total_q, n_seqs, max_rows, max_blocks, num_pages, h_q, h_kv,
                                  head_dim, page_size, scale, sliding_window, dtype, nullptr, 0,
                                  max_kv, (hipStream_t)stream, 0, nullptr);
}

extern "C" int vx_paged_decode_attention(const void *q, const void *k_pool, const void *v_pool,
                                         const uint32_t *block_table, const uint32_t *kv_lens,
                                         void *out, int64_t n, int64_t max_blocks, int64_t num_pages,
                                         int64_t h_q, int64_t h_kv, int64_t head_dim,
                                         int64_t page_size, float scale, uint32_t sliding_window,
                                         int dtype, void *stream) {
    VX_TRY(check_attn_shapes(h_q, h_kv, head_dim, dtype));
    if (n == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(q && k_pool && v_pool && block_table && kv_lens && out, "paged_decode_attention: null tensor");
    VX_REQUIRE(max_blocks > 0 && num_pages > 0 && page_size > 0, "paged_decode_attention: empty pool");
    return paged_attention_launch(q, k_pool, v_pool, block_table, nullptr, kv_lens, nullptr, out, 1, n, n,
                                  1, max_blocks, num_pages, h_q, h_kv, head_dim, page_size, scale,
                                  sliding_window, dtype, nullptr, 0, max_blocks * page_size,
                                  (hipStream_t)stream, 0, nullptr);
}
