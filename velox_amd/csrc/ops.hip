// Row-wise kernels of the verify path, gfx950: embedding, RMSNorm, fused
// q/k-norm + RoPE + KV write, the RoPE / scatter drop-ins, and acceptance.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "vx_common.h"

namespace vx {

// ===========================================================================
// embedding + norms (qwen3.rs:998, :393-394, :923-928, :965; candle RmsNorm)
// ===========================================================================

// h[r, :] = round_T(embed[ids[r], :]); embed is stored in T already.
constexpr int kMaxFusedSplits = 8;  // split partials a fused finish reads

// Sum over the workgroup (threads = 64 * waves <= 1024), same value in every thread.
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < nw; w++) t += red[w];
    return t;
}

// Eight bf16 values (one 16-byte piece of a row) -> floats.
__device__ __forceinline__ void bf16x8_unpack(uint4 v, float (&f)[8]) {
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[2 * e] = __uint_as_float(u[e] << 16);
        f[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
    }
}

// y = round_bf16(x / m * w) for the thread's eight columns, m = sqrt(mean(x^2) + eps),
// stored as f16 (exact carrier of the bf16 value) or bf16.
__device__ __forceinline__ uint4 rms_apply8(const float (&x)[8], uint4 wv, float m, int out_dt) {
    float w[8];
    bf16x8_unpack(wv, w);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float a = round_to<VX_BF16>(x[2 * e] / m * w[2 * e]);
        const float b = round_to<VX_BF16>(x[2 * e + 1] / m * w[2 * e + 1]);
        o[e] = out_dt == VX_F16 ? ((uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16))
                                : ((uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// y = round_bf16(x / sqrt(mean(x^2) + eps) * w) (candle RmsNorm in bf16), x, w
// bf16, y as f16 carrier or bf16.  Rows optionally gathered through row_idx
// (the last row per sequence, or token ids into the embedding table, read
// idx_stride apart: indices clamp to src_rows - 1), and the gathered rows
// optionally copied to xcopy
// (the embedding lookup, qwen3.rs:998, fused with the first layer's norm).
// One workgroup per row, one thread per 8 columns; the row and the weights
// are requested together up front.
__global__ __launch_bounds__(1024) void rmsnorm_bf16_kernel(const uint16_t *x, const uint16_t *w, uint16_t *y,
                                                           const uint32_t *row_idx, int H, float eps, int out_dt,
                                                           int64_t src_rows, uint16_t *xcopy, int64_t idx_stride) {
    __shared__ float red[16];
    const int r = blockIdx.x;
    const int i = threadIdx.x;
    const bool live = i < H / 8;
    const int64_t src_r = row_idx ? std::min<int64_t>(row_idx[(int64_t)r * idx_stride], src_rows - 1) : r;
    const uint4 xv = live ? ((const uint4 *)(x + src_r * H))[i] : make_uint4(0u, 0u, 0u, 0u);
    if (xcopy && live) ((uint4 *)(xcopy + (int64_t)r * H))[i] = xv;
    const uint4 wv = live ? ((const uint4 *)w)[i] : make_uint4(0u, 0u, 0u, 0u);
    float f[8];
    bf16x8_unpack(xv, f);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) s += f[e] * f[e];
    const float m = sqrtf(block_sum(s, red) / (float)H + eps);
    if (live) ((uint4 *)(y + (int64_t)r * H))[i] = rms_apply8(f, wv, m, out_dt);
}

// A projection's finish fused with the next RMSNorm, one workgroup per row:
//   h[r, :] = round_bf16(h[r, :] + round_bf16(acc_scale * sum_sp partial[sp][r][:]))
// (the RESIDUAL epilogue, partials summed in split order), written back as
// bf16; then, when ln is given, y = RMSNorm(h) * ln as rmsnorm_bf16_kernel.
__global__ __launch_bounds__(1024) void residual_rmsnorm_kernel(const float *partial, int splits, float acc_scale,
                                                               uint16_t *hrow, const uint16_t *ln, uint16_t *y,
                                                               int rows, int H, float eps, int out_dt) {
    __shared__ float red[16];
    const int r = blockIdx.x;
    const int i = threadIdx.x;
    const bool live = i < H / 8;
    uint4 *hr = (uint4 *)(hrow + (int64_t)r * H);
    const uint4 old = live ? hr[i] : make_uint4(0u, 0u, 0u, 0u);
    const uint4 wv = (live && ln) ? ((const uint4 *)ln)[i] : make_uint4(0u, 0u, 0u, 0u);
    float4 p[kMaxFusedSplits][2];
#pragma unroll
    for (int sp = 0; sp < kMaxFusedSplits; sp++) {
        if (live && sp < splits) {
            const float4 *pp = (const float4 *)(partial + ((int64_t)sp * rows + r) * H + 8 * i);
            p[sp][0] = pp[0];
            p[sp][1] = pp[1];
        } else {
            p[sp][0] = p[sp][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < kMaxFusedSplits; sp++) {
        if (sp < splits) {
            acc[0] += p[sp][0].x; acc[1] += p[sp][0].y; acc[2] += p[sp][0].z; acc[3] += p[sp][0].w;
            acc[4] += p[sp][1].x; acc[5] += p[sp][1].y; acc[6] += p[sp][1].z; acc[7] += p[sp][1].w;
        }
    }
    float hv[8];
    bf16x8_unpack(old, hv);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; e++) hv[e] = round_to<VX_BF16>(hv[e] + round_to<VX_BF16>(acc[e] * acc_scale));
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = (uint32_t)f32_to_bf16_bits(hv[2 * e]) | ((uint32_t)f32_to_bf16_bits(hv[2 * e + 1]) << 16);
    if (live) hr[i] = make_uint4(o[0], o[1], o[2], o[3]);
    if (!ln) return;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) s += hv[e] * hv[e];
    const float m = sqrtf(block_sum(s, red) / (float)H + eps);
    if (live) ((uint4 *)(y + (int64_t)r * H))[i] = rms_apply8(hv, wv, m, out_dt);
}

// Per (row, head), one wave: q/k heads get the per-head RMSNorm
// (qwen3.rs:435-454) and RoPE at rope_pos[row] (MSL :209-241, tables in
// bf16); q goes to qout and k, v are written into the pools at
// (page_ids[row], slots[row]) (MSL :251-279), all in the pool dtype (f16
// pools carry the bf16-rounded values exactly).  Lane j holds the RoPE pair
// (j, j + D/2).  With PARTIAL the qkv row is the sum of the projection's f32
// split partials [splits][rows][N] in split order, rounded to bf16 as the
// projection's store would (the projection's finish fused here).
template <bool PARTIAL>
__global__ __launch_bounds__(256) void qk_rope_scatter_kernel(
    const uint16_t *qkv, const float *partial, int splits, const uint16_t *qn_w, const uint16_t *kn_w,
    const uint16_t *cos_t, const uint16_t *sin_t, const uint32_t *rope_pos, const uint32_t *page_ids,
    const uint32_t *slots, uint16_t *qout, uint16_t *k_pool, uint16_t *v_pool, int rows, int HQ, int HK,
    int D, int ps, float eps, int kv_dt) {
    const int NH = HQ + 2 * HK;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (gw >= rows * NH) return;
    const int r = gw / NH;
    const int h = gw - r * NH;
    const int QW = HQ * D, KW = HK * D, N = QW + 2 * KW;
    const uint16_t *row = qkv + (int64_t)r * N;
    auto val = [&](int c) -> float {
        if constexpr (PARTIAL) {
            float pv[kMaxFusedSplits];
#pragma unroll
            for (int sp = 0; sp < kMaxFusedSplits; sp++)
                pv[sp] = sp < splits ? partial[((int64_t)sp * rows + r) * N + c] : 0.f;
            float acc = 0.f;
#pragma unroll
            for (int sp = 0; sp < kMaxFusedSplits; sp++)
                if (sp < splits) acc += pv[sp];
            return round_to<VX_BF16>(acc);
        } else {
            return bf16_bits_to_f32(row[c]);
        }
    };
    const int half = D / 2;
    const int64_t page = page_ids[r];
    const int slot = (int)slots[r];
    if (h >= HQ + HK) {  // v head: plain copy
        const int hv = h - HQ - HK;
        const int c0 = QW + KW + hv * D;
        uint16_t *dst = v_pool + ((page * HK + hv) * ps + slot) * (int64_t)D;
        for (int i = lane; i < D; i += 64) {
            const float v = val(c0 + i);
            dst[i] = kv_dt == VX_F16 ? f32_to_f16_bits(v) : f32_to_bf16_bits(v);
        }
        return;
    }
    const uint32_t pos = rope_pos[r];
    const bool is_q = h < HQ;
    const int c0 = is_q ? h * D : QW + (h - HQ) * D;
    const uint16_t *nw = is_q ? qn_w : kn_w;
    // per-head RMSNorm over D: lane holds pairs (j, j + half) for j = lane, lane + 64, ...
    constexpr int kMaxPairs = 2;  // D <= 256
    float x1[kMaxPairs], x2[kMaxPairs];
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < kMaxPairs; p++) {
        const int j = lane + 64 * p;
        x1[p] = j < half ? val(c0 + j) : 0.f;
        x2[p] = j < half ? val(c0 + j + half) : 0.f;
        ss += x1[p] * x1[p];
        ss += x2[p] * x2[p];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float m = sqrtf(ss / (float)D + eps);
    uint16_t *dst = is_q ? qout + ((int64_t)r * HQ + h) * D
                         : k_pool + ((page * HK + (h - HQ)) * ps + slot) * (int64_t)D;
#pragma unroll
    for (int p = 0; p < kMaxPairs; p++) {
        const int j = lane + 64 * p;
        if (j >= half) break;
        const float a = round_to<VX_BF16>(x1[p] / m * bf16_bits_to_f32(nw[j]));
        const float b = round_to<VX_BF16>(x2[p] / m * bf16_bits_to_f32(nw[j + half]));
        const float c = bf16_bits_to_f32(cos_t[(int64_t)pos * half + j]);
        const float s = bf16_bits_to_f32(sin_t[(int64_t)pos * half + j]);
        const float y1 = round_to<VX_BF16>(__fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s)));
        const float y2 = round_to<VX_BF16>(__fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c)));
        if (kv_dt == VX_F16) {
            dst[j] = f32_to_f16_bits(y1);
            dst[j + half] = f32_to_f16_bits(y2);
        } else {
            dst[j] = f32_to_bf16_bits(y1);
            dst[j + half] = f32_to_bf16_bits(y2);
        }
    }
}

// ===========================================================================
// drop-in RoPE / scatter (metal_kernels.rs MSL :209-241, :251-279)
// ===========================================================================
template <int DT>
__global__ void rope_kernel(void *x, const void *cos_t, const void *sin_t, const uint32_t *offsets,
                            int64_t n, int64_t h, int64_t half) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t tot = n * h * half;
    if (idx >= tot) return;
    const int64_t dp = idx % half;
    const int64_t hh = (idx / half) % h;
    const int64_t r = idx / (half * h);
    const int64_t off = offsets[r];
    const int64_t base = (r * h + hh) * 2 * half;
    const float x1 = ld_elem<DT>(x, base + dp);
    const float x2 = ld_elem<DT>(x, base + dp + half);
    const float c = ld_elem<DT>(cos_t, off * half + dp);
    const float s = ld_elem<DT>(sin_t, off * half + dp);
    st_elem<DT>(x, base + dp, __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s)));
    st_elem<DT>(x, base + dp + half, __fadd_rn(__fmul_rn(x1, s), __fmul_rn(x2, c)));
}

__global__ void scatter_kernel(uint8_t *pool, const uint8_t *values, const uint32_t *page_ids,
                               const uint32_t *slots, int64_t n, int64_t h, int64_t ps,
                               int64_t row_bytes, int64_t num_pages) {
    // one block per (row, head); row_bytes = d * elem
    const int64_t r = blockIdx.x / h;
    const int64_t hh = blockIdx.x % h;
    const int64_t page = page_ids[r];
    const int64_t slot = slots[r];
    if (page >= num_pages || slot >= ps) return;
    const uint8_t *src = values + (r * h + hh) * row_bytes;
    uint8_t *dst = pool + ((page * h + hh) * ps + slot) * row_bytes;
    for (int64_t i = threadIdx.x * 4; i < row_bytes; i += blockDim.x * 4)
        *(uint32_t *)(dst + i) = *(const uint32_t *)(src + i);
}

// ===========================================================================
// argmax / acceptance
// ===========================================================================
constexpr int kArgChunk = 8192;
constexpr int kSmThreads = 256;
constexpr int kSmChunk = 8192;  // softmax statistics chunk (matches the host definition)
constexpr int kSmSub = 256;     // residual-sampling sub-chunk

struct ArgBest {
    float v;
    uint32_t i;
};
__device__ __forceinline__ ArgBest arg_better(ArgBest a, ArgBest b) {
    // larger value wins; equal values: smaller index; "none" is (-inf, ~0u)
    if (b.v > a.v) return b;
    if (a.v > b.v) return a;
    return b.i < a.i ? b : a;
}

template <int DT>
__device__ ArgBest chunk_argmax(const void *row, int64_t lo, int64_t hi, float *sv, uint32_t *si) {
    ArgBest best = {-__builtin_inff(), 0xffffffffu};
    for (int64_t j = lo + threadIdx.x; j < hi; j += blockDim.x) {
        const float v = ld_elem<DT>(row, j);
        if (v > best.v) {  // strict: the first (smallest) index per thread wins ties; NaN never wins
            best.v = v;
            best.i = (uint32_t)j;
        }
    }
    sv[threadIdx.x] = best.v;
    si[threadIdx.x] = best.i;
    __syncthreads();
    for (int st = blockDim.x / 2; st > 0; st >>= 1) {
        if ((int)threadIdx.x < st) {
            ArgBest o = arg_better({sv[threadIdx.x], si[threadIdx.x]}, {sv[threadIdx.x + st], si[threadIdx.x + st]});
            sv[threadIdx.x] = o.v;
            si[threadIdx.x] = o.i;
        }
        __syncthreads();
    }
    ArgBest r = {sv[0], si[0]};
    __syncthreads();
    return r;
}

struct AcceptArgs {
    const void *logits;
    int64_t vocab;
    int rows_per_group;  // rows belonging to one sequence
    int n_chunks;        // argmax chunks per row
    float *pv;           // partial values [rows, n_chunks]
    uint32_t *pi;        // partial indices
    int mode;            // 0 argmax rows, 1 greedy chain, 2 tree
    const uint32_t *cand;  // chain: [B, k]; tree: node tokens [B, R]
    int k;
    int32_t *accepted;
    uint32_t *tokens;    // chain: [B, k+1]; tree: [B, R]
    int32_t *path;       // tree: [B, R]
    uint32_t *argmax_out;  // optional [rows]
    uint32_t *next_ids;    // optional (mode 0): argmax also written here ([rows], stride next_stride)
    int64_t next_stride;
    int parents[64];
};

// Pass 1: (max, first index) of every 8192-wide chunk of every row.
template <int DT>
__global__ __launch_bounds__(256) void argmax_partial_kernel(AcceptArgs a) {
    __shared__ float sv[256];
    __shared__ uint32_t si[256];
    const int64_t row = blockIdx.x / a.n_chunks;
    const int chunk = blockIdx.x % a.n_chunks;
    const int64_t lo = (int64_t)chunk * kArgChunk;
    const int64_t hi = min(a.vocab, lo + kArgChunk);
    const void *rowp = (const char *)a.logits + row * a.vocab * (DT == VX_F32 ? 4 : 2);
    const ArgBest cbest = chunk_argmax<DT>(rowp, lo, hi, sv, si);
    if (threadIdx.x == 0) {
        a.pv[row * a.n_chunks + chunk] = cbest.v;
        a.pi[row * a.n_chunks + chunk] = cbest.i;
    }
}

// Pass 2: one block per group (sequence): combine chunk partials of each row
// in chunk order, then the acceptance walk on thread 0.
// The partials never hold NaN (it never wins a chunk), so arg_better is a
// total order on them and the 64 lanes may combine a row's chunks strided and
// then by butterfly: the same winner as the sequential scan.
// One wave per row of the group (up to kAcceptWaves, then strided): the
// row's partials are requested 24 per lane at a time (one memory round trip
// for up to 1536 partials, the LM head's 1187), and rows run in parallel.
constexpr int kAcceptWaves = 8;
__global__ __launch_bounds__(64 * kAcceptWaves) void accept_finish_kernel(AcceptArgs a) {
    __shared__ uint32_t am[64];
    const int64_t grp = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int waves = blockDim.x >> 6;
    for (int rr = threadIdx.x >> 6; rr < a.rows_per_group; rr += waves) {
        const int64_t rw = grp * a.rows_per_group + rr;
        ArgBest best = {-__builtin_inff(), 0xffffffffu};
        for (int c0 = lane; c0 < a.n_chunks; c0 += 64 * 24) {
            float v[24];
            uint32_t ix[24];
#pragma unroll
            for (int u = 0; u < 24; u++) {
                const int c = c0 + 64 * u;
                v[u] = c < a.n_chunks ? a.pv[rw * a.n_chunks + c] : -__builtin_inff();
                ix[u] = c < a.n_chunks ? a.pi[rw * a.n_chunks + c] : 0xffffffffu;
            }
#pragma unroll
            for (int u = 0; u < 24; u++) best = arg_better(best, {v[u], ix[u]});
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            best = arg_better(best, {__shfl_xor(best.v, o), (uint32_t)__shfl_xor((int)best.i, o)});
        if (lane == 0) {
            const uint32_t idx = best.i == 0xffffffffu ? 0u : best.i;
            am[rr] = idx;
            if (a.argmax_out) a.argmax_out[rw] = idx;
            if (a.mode == 0 && a.next_ids) a.next_ids[rw * a.next_stride] = idx;
        }
    }
    __syncthreads();
    if (threadIdx.x != 0 || a.mode == 0) return;
    const int64_t b = grp;
    if (a.mode == 1) {  // spec.rs:284-292
        int acc = 0;
        while (acc < a.k && a.cand[b * a.k + acc] == am[acc]) acc++;
        for (int i = 0; i < acc; i++) a.tokens[b * (a.k + 1) + i] = a.cand[b * a.k + i];
        a.tokens[b * (a.k + 1) + acc] = am[acc];
        a.accepted[b] = acc;
    } else {  // tree walk from the root
        const int R = a.rows_per_group;
        int cur = 0, acc = 0;
        a.path[b * R] = 0;
        for (;;) {
            const uint32_t t = am[cur];
            int nxt = -1;
            for (int j = cur + 1; j < R; j++)
                if (a.parents[j] == cur && a.cand[b * R + j] == t) {
                    nxt = j;
                    break;
                }
            if (nxt < 0) break;
            a.tokens[b * R + acc] = t;
            acc++;
            a.path[b * R + acc] = nxt;
            cur = nxt;
        }
        a.tokens[b * R + acc] = am[cur];
        a.accepted[b] = acc;
    }
}

// ---- stochastic acceptance ------------------------------------------------
// Row statistics with the fixed structure shared with the host definition:
// per chunk of 8192, 256 strided thread partials folded by a stride-halving
// tree; chunk (max, sum) pairs combined in chunk order by the consumer.
template <int DT>
__global__ __launch_bounds__(256) void softmax_stats_kernel(const void *logits, int64_t vocab,
                                                            float inv_t, float *cm, float *cz,
                                                            int n_chunks) {
    __shared__ float red[256];
    const int64_t row = blockIdx.x / n_chunks;
    const int chunk = blockIdx.x % n_chunks;
    const int64_t lo = (int64_t)chunk * kSmChunk;
    const int64_t hi = min(vocab, lo + kSmChunk);
    const void *r = (const char *)logits + row * vocab * (DT == VX_F32 ? 4 : 2);
    float m = -__builtin_inff();
    for (int64_t j = lo + threadIdx.x; j < hi; j += 256) m = fmaxf(m, ld_elem<DT>(r, j));
    red[threadIdx.x] = m;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if ((int)threadIdx.x < st) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + st]);
        __syncthreads();
    }
    m = red[0];
    __syncthreads();
    // a chunk with no finite maximum holds no probability mass
    float s = 0.f;
    if (m != -__builtin_inff())
        for (int64_t j = lo + threadIdx.x; j < hi; j += 256)
            s = __fadd_rn(s, vx_detexp(__fmul_rn(__fsub_rn(ld_elem<DT>(r, j), m), inv_t)));
    red[threadIdx.x] = s;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if ((int)threadIdx.x < st) red[threadIdx.x] = __fadd_rn(red[threadIdx.x], red[threadIdx.x + st]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        cm[row * n_chunks + chunk] = m;
        cz[row * n_chunks + chunk] = red[0];
    }
}

__device__ __forceinline__ void combine_stats(const float *cm, const float *cz, int n_chunks,
                                              float inv_t, float &M, float &Z) {
    M = -__builtin_inff();
    for (int c = 0; c < n_chunks; c++) M = fmaxf(M, cm[c]);
    Z = 0.f;
    for (int c = 0; c < n_chunks; c++)
        if (cm[c] != -__builtin_inff()) Z = __fadd_rn(Z, __fmul_rn(cz[c], vx_detexp(__fmul_rn(__fsub_rn(cm[c], M), inv_t))));
}

template <int DT>
__device__ __forceinline__ float resid_elem(const void *lt, float mt, float zt, const void *ld,
                                            float md, float zd, float inv_t, int64_t j) {
    // a row with no finite logit has no mass anywhere
    const float p = mt == -__builtin_inff() ? 0.f : __fdiv_rn(vx_detexp(__fmul_rn(__fsub_rn(ld_elem<DT>(lt, j), mt), inv_t)), zt);
    if (!ld) return p;
    const float q = md == -__builtin_inff() ? 0.f : __fdiv_rn(vx_detexp(__fmul_rn(__fsub_rn(ld_elem<DT>(ld, j), md), inv_t)), zd);
    const float d = __fsub_rn(p, q);
    return d > 0.f ? d : 0.f;
}

// ---- residual / softmax draws ----------------------------------------------
// Inverse-CDF draw over r_j (p_j, or max(0, p_j - q_j) for a rejection) with
// the hierarchical prefix order shared with the host definition: 256-element
// sub-chunks summed sequentially in index order, 32 sub-chunk sums per
// 8192-element chunk summed in order, chunk sums in order; the walk descends
// chunk -> sub-chunk -> element.  If rounding leaves the walk short inside a
// chunk, the draw is the chunk's last index with r_j > 0; if it never crosses
// the target, the row's last such index (0 if none).
//
// Two launches per batch of draws: resid_chunk_kernel (one workgroup per
// draw and chunk: r_j staged in LDS from coalesced loads, the 32 sub-chunk
// sums, the chunk sum, the chunk's last positive index) and resid_walk_kernel
// (one workgroup per draw: the descent, with the selected sub-chunk's r_j
// recomputed in parallel and walked by one lane).
constexpr int kSubPerChunk = kSmChunk / kSmSub;  // 32
constexpr int kMaxChunks = 32;                    // vocab <= 262144

struct DrawDesc {
    int64_t trow;  // row of the target (or sampled) logits
    int64_t drow;  // row of the draft logits, -1 = plain softmax draw
    float mt, zt, md, zd, u;
    int64_t out;   // index of the drawn token in the token output
};

struct DrawArgs {
    const void *tl, *dl;
    const float *uni;    // SAMPLE: uniforms[row * ustride]
    int64_t ustride;
    const float *cm, *cz;  // SAMPLE: chunk statistics of each row
    int n_chunks;
    int64_t vocab;
    float inv_t;
    DrawDesc *desc;  // [draws]
    float *ss;       // [draws, n_chunks * 32] sub-chunk sums
    float *cs;       // [draws, n_chunks] chunk sums
    int32_t *lastpos;  // [draws, n_chunks] last index with r_j > 0, -1 = none
    uint32_t *out;     // token output (SAMPLE: [draws]; accept: tokens indexed by desc.out)
    uint32_t *next_ids;
    int64_t next_stride;
};

template <int DT>
__device__ __forceinline__ const void *row_ptr(const void *base, int64_t row, int64_t vocab) {
    return (const char *)base + row * vocab * (DT == VX_F32 ? 4 : 2);
}

// SAMPLE: draw d reads row d; its statistics are combined here and the
// descriptor is written by chunk 0's workgroup for the walk.
template <int DT, bool SAMPLE>
__global__ __launch_bounds__(256) void resid_chunk_kernel(DrawArgs a) {
    __shared__ float rb[kSmSub * (kSubPerChunk + 1)];  // [position][sub-chunk], padded: conflict-free both ways
    __shared__ float sub[kSubPerChunk];
    __shared__ DrawDesc sd;
    __shared__ int s_last;
    const int nch = a.n_chunks;
    const int64_t d = blockIdx.x / nch;
    const int c = blockIdx.x % nch;
    const int tid = threadIdx.x;
    if (tid == 0) {
        DrawDesc x;
        if (SAMPLE) {
            float M, Z;
            combine_stats(a.cm + d * nch, a.cz + d * nch, nch, a.inv_t, M, Z);
            x = {d, -1, M, Z, 0.f, 1.f, a.uni[d * a.ustride], d};
            if (c == 0) a.desc[d] = x;
        } else {
            x = a.desc[d];
        }
        sd = x;
        s_last = -1;
    }
    __syncthreads();
    const void *lt = row_ptr<DT>(a.tl, sd.trow, a.vocab);
    const void *ld = sd.drow >= 0 ? row_ptr<DT>(a.dl, sd.drow, a.vocab) : nullptr;
    const float mt = sd.mt, zt = sd.zt, md = sd.md, zd = sd.zd;
    const int64_t lo = (int64_t)c * kSmChunk;
    const int n = (int)min((int64_t)kSmChunk, a.vocab - lo);
    int my_last = -1;
#pragma unroll 4
    for (int i = 0; i < kSubPerChunk; i++) {
        const int jl = i * kSmSub + tid;
        float r = 0.f;
        if (jl < n) {
            r = resid_elem<DT>(lt, mt, zt, ld, md, zd, a.inv_t, lo + jl);
            if (r > 0.f) my_last = (int)(lo + jl);
        }
        rb[tid * (kSubPerChunk + 1) + i] = r;
    }
    atomicMax(&s_last, my_last);
    __syncthreads();
    if (tid < kSubPerChunk) {
        const int cnt = max(0, min(kSmSub, n - tid * kSmSub));
        float s = 0.f;
        for (int p = 0; p < cnt; p++) s = __fadd_rn(s, rb[p * (kSubPerChunk + 1) + tid]);
        sub[tid] = s;
        a.ss[(d * nch + c) * kSubPerChunk + tid] = s;
    }
    __syncthreads();
    if (tid == 0) {
        float s = 0.f;
        for (int i = 0; i < kSubPerChunk; i++) s = __fadd_rn(s, sub[i]);
        a.cs[d * nch + c] = s;
        a.lastpos[d * nch + c] = s_last;
    }
}

template <int DT, bool SAMPLE>
__global__ __launch_bounds__(256) void resid_walk_kernel(DrawArgs a) {
    __shared__ float s_cs[kMaxChunks];
    __shared__ int s_lp[kMaxChunks];
    __shared__ float s_ss[kSubPerChunk];
    __shared__ float rb[kSmSub];
    __shared__ int s_c, s_s;
    __shared__ float s_run, s_target;
    __shared__ uint32_t s_result;
    const int nch = a.n_chunks;
    const int64_t d = blockIdx.x;
    const int tid = threadIdx.x;
    const DrawDesc x = a.desc[d];
    if (tid < nch) {
        s_cs[tid] = a.cs[d * nch + tid];
        s_lp[tid] = a.lastpos[d * nch + tid];
    }
    __syncthreads();
    if (tid == 0) {
        float total = 0.f;
        int last = -1;
        for (int c = 0; c < nch; c++) {
            total = __fadd_rn(total, s_cs[c]);
            last = max(last, s_lp[c]);
        }
        const float target = __fmul_rn(x.u, total);
        float run = 0.f;
        int sel = -1;
        for (int c = 0; c < nch; c++) {
            if (__fadd_rn(run, s_cs[c]) > target) {
                sel = c;
                break;
            }
            run = __fadd_rn(run, s_cs[c]);
        }
        s_c = sel;
        s_run = run;
        s_target = target;
        s_result = last < 0 ? 0u : (uint32_t)last;
    }
    __syncthreads();
    const int c = s_c;
    if (c >= 0) {  // uniform across the block
        if (tid < kSubPerChunk) s_ss[tid] = a.ss[(d * nch + c) * kSubPerChunk + tid];
        __syncthreads();
        if (tid == 0) {
            float run = s_run;
            int sel = -1;
            for (int i = 0; i < kSubPerChunk; i++) {
                if (__fadd_rn(run, s_ss[i]) > s_target) {
                    sel = i;
                    break;
                }
                run = __fadd_rn(run, s_ss[i]);
            }
            s_s = sel;
            s_run = run;
        }
        __syncthreads();
        const int s = s_s;
        const int64_t lo = ((int64_t)c * kSubPerChunk + max(s, 0)) * kSmSub;
        const int cnt = (int)min((int64_t)kSmSub, a.vocab - lo);
        if (s >= 0 && tid < cnt) {
            const void *lt = row_ptr<DT>(a.tl, x.trow, a.vocab);
            const void *ld = x.drow >= 0 ? row_ptr<DT>(a.dl, x.drow, a.vocab) : nullptr;
            rb[tid] = resid_elem<DT>(lt, x.mt, x.zt, ld, x.md, x.zd, a.inv_t, lo + tid);
        }
        __syncthreads();
        if (tid == 0) {
            int64_t found = -1;
            if (s >= 0) {
                float run = s_run;
                for (int p = 0; p < cnt; p++) {
                    run = __fadd_rn(run, rb[p]);
                    if (run > s_target) {
                        found = lo + p;
                        break;
                    }
                }
            }
            if (found < 0) found = s_lp[c];
            if (found >= 0) s_result = (uint32_t)found;
        }
    }
    if (tid == 0) {
        const uint32_t t = s_result;
        if (SAMPLE) {
            a.out[d] = t;
            if (a.next_ids) a.next_ids[d * a.next_stride] = t;
        } else {
            a.out[x.out] = t;
        }
    }
}

// One lane per sequence: the accept/reject walk over the k candidates; the
// accepted candidates are written, and the descriptor of the one draw that
// follows (residual row at the first rejection, else the bonus row).
// Draft row of (b, i): b * k + i, or i * batch + b when draft_step_major.
__global__ __launch_bounds__(64) void stochastic_walk_kernel(
    const void *tl, const void *dl, int ldt, const uint32_t *cand, const float *uni, const float *cm_t,
    const float *cz_t, const float *cm_d, const float *cz_d, int n_chunks, int64_t vocab, int k, int64_t batch,
    int draft_step_major, float inv_t, int32_t *accepted, uint32_t *tokens, DrawDesc *desc) {
    const int64_t b = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (b >= batch) return;
    const size_t esz = ldt == VX_F32 ? 4 : 2;
    for (int i = 0; i < k; i++) {
        const int64_t trow = b * (k + 1) + i;
        const int64_t drow = draft_step_major ? i * batch + b : b * k + i;
        float mt, zt, md, zd;
        combine_stats(cm_t + trow * n_chunks, cz_t + trow * n_chunks, n_chunks, inv_t, mt, zt);
        combine_stats(cm_d + drow * n_chunks, cz_d + drow * n_chunks, n_chunks, inv_t, md, zd);
        const uint32_t c = cand[b * k + i];
        const void *tr = (const char *)tl + trow * vocab * esz;
        const void *dr = (const char *)dl + drow * vocab * esz;
        float lt_c, ld_c;
        if (ldt == VX_BF16) {
            lt_c = ld_elem<VX_BF16>(tr, c);
            ld_c = ld_elem<VX_BF16>(dr, c);
        } else if (ldt == VX_F16) {
            lt_c = ld_elem<VX_F16>(tr, c);
            ld_c = ld_elem<VX_F16>(dr, c);
        } else {
            lt_c = ld_elem<VX_F32>(tr, c);
            ld_c = ld_elem<VX_F32>(dr, c);
        }
        const float p = mt == -__builtin_inff() ? 0.f : __fdiv_rn(vx_detexp(__fmul_rn(__fsub_rn(lt_c, mt), inv_t)), zt);
        const float q = md == -__builtin_inff() ? 0.f : __fdiv_rn(vx_detexp(__fmul_rn(__fsub_rn(ld_c, md), inv_t)), zd);
        const float ratio = __fdiv_rn(p, q);
        const float acc = ratio < 1.0f ? ratio : 1.0f;
        if (!(uni[trow * 4 + 1] < acc)) {
            desc[b] = {trow, drow, mt, zt, md, zd, uni[trow * 4 + 2], trow};
            accepted[b] = i;
            return;
        }
        tokens[trow] = c;
    }
    const int64_t trow = b * (k + 1) + k;
    float mt, zt;
    combine_stats(cm_t + trow * n_chunks, cz_t + trow * n_chunks, n_chunks, inv_t, mt, zt);
    desc[b] = {trow, -1, mt, zt, 0.f, 1.f, uni[trow * 4 + 2], trow};
    accepted[b] = k;
}
}  // namespace vx

using namespace vx;

namespace vx {

constexpr size_t kAccCounterBytes = 65536;

size_t accept_workspace_bytes(int64_t rows, int64_t vocab) {
    const int64_t nch = vx_cdiv(vocab, kArgChunk);
    return kAccCounterBytes + (size_t)rows * nch * 8 * 2 + 256;
}

int argmax_accept_launch(const void *logits, int ldt, int64_t rows, int64_t vocab, int mode,
                         int rows_per_group, const uint32_t *cand, int k, int32_t *accepted,
                         uint32_t *tokens, int32_t *path, const int32_t *parents, uint32_t *argmax_out,
                         uint32_t *next_ids, int64_t next_stride, void *ws, size_t ws_bytes,
                         hipStream_t st) {
    VX_REQUIRE(vocab > 0 && rows > 0, "argmax: empty logits");
    AcceptArgs a{};
    a.logits = logits;
    a.vocab = vocab;
    a.rows_per_group = rows_per_group;
    a.n_chunks = (int)vx_cdiv(vocab, kArgChunk);
    const size_t need = accept_workspace_bytes(rows, vocab);
    if (!ws) {
        VX_TRY(stream_workspace(st, need, &ws));
    } else if (ws_bytes < need) {
        return set_error("accept: workspace too small");
    }
    VX_REQUIRE(rows_per_group >= 1 && rows_per_group <= 64 && rows % rows_per_group == 0,
               "accept: rows per sequence must be 1..64");
    a.pv = (float *)((char *)ws + kAccCounterBytes);
    a.pi = (uint32_t *)((char *)a.pv + (size_t)rows * a.n_chunks * 4);
    a.mode = mode;
    a.cand = cand;
    a.k = k;
    a.accepted = accepted;
    a.tokens = tokens;
    a.path = path;
    a.argmax_out = argmax_out;
    a.next_ids = next_ids;
    a.next_stride = next_stride;
    if (parents)
        for (int i = 0; i < rows_per_group && i < 64; i++) a.parents[i] = parents[i];
    dim3 grid((unsigned)(rows * a.n_chunks));
    if (ldt == VX_BF16)
        hipLaunchKernelGGL(argmax_partial_kernel<VX_BF16>, grid, dim3(256), 0, st, a);
    else if (ldt == VX_F16)
        hipLaunchKernelGGL(argmax_partial_kernel<VX_F16>, grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(argmax_partial_kernel<VX_F32>, grid, dim3(256), 0, st, a);
    hipLaunchKernelGGL(accept_finish_kernel, dim3((unsigned)(rows / rows_per_group)),
                       dim3(64 * std::min(rows_per_group, kAcceptWaves)), 0, st, a);
    VX_HIP(hipGetLastError());
    return 0;
}

// Greedy argmax / acceptance from (value, first index) partials that the LM
// head's GEMM epilogue wrote ([rows, n_chunks], one per 128 columns): the
// first pass over the logits is skipped.
int argmax_accept_partials_launch(const float *pv, const uint32_t *pi, int n_chunks, int64_t rows, int mode,
                                  int rows_per_group, const uint32_t *cand, int k, int32_t *accepted,
                                  uint32_t *tokens, uint32_t *next_ids, int64_t next_stride, hipStream_t st) {
    VX_REQUIRE(rows > 0 && n_chunks > 0, "argmax: empty partials");
    VX_REQUIRE(rows_per_group >= 1 && rows_per_group <= 64 && rows % rows_per_group == 0,
               "accept: rows per sequence must be 1..64");
    VX_REQUIRE(mode == 0 || mode == 1, "accept: partials serve greedy argmax and chain acceptance");
    AcceptArgs a{};
    a.rows_per_group = rows_per_group;
    a.n_chunks = n_chunks;
    a.pv = (float *)pv;
    a.pi = (uint32_t *)pi;
    a.mode = mode;
    a.cand = cand;
    a.k = k;
    a.accepted = accepted;
    a.tokens = tokens;
    a.next_ids = next_ids;
    a.next_stride = next_stride;
    hipLaunchKernelGGL(accept_finish_kernel, dim3((unsigned)(rows / rows_per_group)),
                       dim3(64 * std::min(rows_per_group, kAcceptWaves)), 0, st, a);
    VX_HIP(hipGetLastError());
    return 0;
}

// Workspace of the stochastic paths, after the arrival-counter region (so
// argmax / accept launches sharing the workspace keep their zeroed
// counters): chunk statistics of `stat_rows` rows, then `draws` descriptors,
// sub-chunk sums, chunk sums and last positive indices.
struct StochLayout {
    float *cm, *cz;
    DrawDesc *desc;
    float *ss, *cs;
    int32_t *lastpos;
};

static size_t stoch_layout(void *ws, int64_t stat_rows, int64_t draws, int nch, StochLayout *L) {
    size_t off = kAccCounterBytes;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = (off + bytes + 255) & ~(size_t)255;
        return (char *)ws + at;
    };
    char *cm = take((size_t)stat_rows * nch * 4);
    char *cz = take((size_t)stat_rows * nch * 4);
    char *desc = take((size_t)draws * sizeof(DrawDesc));
    char *ss = take((size_t)draws * nch * kSubPerChunk * 4);
    char *cs = take((size_t)draws * nch * 4);
    char *lp = take((size_t)draws * nch * 4);
    if (L) *L = {(float *)cm, (float *)cz, (DrawDesc *)desc, (float *)ss, (float *)cs, (int32_t *)lp};
    return off;
}

size_t stochastic_workspace_bytes(int64_t rows, int64_t vocab) {
    return stoch_layout(nullptr, rows, rows, (int)vx_cdiv(vocab, kSmChunk), nullptr);
}

template <int DT>
static void launch_stats(const void *lg, int64_t rows, int64_t vocab, float inv_t, float *cm, float *cz,
                         int nch, hipStream_t st) {
    hipLaunchKernelGGL(softmax_stats_kernel<DT>, dim3((unsigned)(rows * nch)), dim3(256), 0, st, lg, vocab,
                       inv_t, cm, cz, nch);
}

static void stats(const void *lg, int ldt, int64_t rows, int64_t vocab, float inv_t, float *cm,
                  float *cz, int nch, hipStream_t st) {
    if (ldt == VX_BF16)
        launch_stats<VX_BF16>(lg, rows, vocab, inv_t, cm, cz, nch, st);
    else if (ldt == VX_F16)
        launch_stats<VX_F16>(lg, rows, vocab, inv_t, cm, cz, nch, st);
    else
        launch_stats<VX_F32>(lg, rows, vocab, inv_t, cm, cz, nch, st);
}

template <int DT, bool SAMPLE>
static void launch_draws_dt(const DrawArgs &a, int64_t draws, hipStream_t st) {
    hipLaunchKernelGGL((resid_chunk_kernel<DT, SAMPLE>), dim3((unsigned)(draws * a.n_chunks)), dim3(256), 0, st, a);
    hipLaunchKernelGGL((resid_walk_kernel<DT, SAMPLE>), dim3((unsigned)draws), dim3(256), 0, st, a);
}

template <bool SAMPLE>
static void launch_draws(const DrawArgs &a, int ldt, int64_t draws, hipStream_t st) {
    if (ldt == VX_BF16)
        launch_draws_dt<VX_BF16, SAMPLE>(a, draws, st);
    else if (ldt == VX_F16)
        launch_draws_dt<VX_F16, SAMPLE>(a, draws, st);
    else
        launch_draws_dt<VX_F32, SAMPLE>(a, draws, st);
}

int sample_rows_launch(const void *logits, int ldt, const float *uni, int64_t ustride, uint32_t *out,
                       int64_t rows, int64_t vocab, float temperature, uint32_t *next_ids,
                       int64_t next_stride, void *ws, size_t ws_bytes, hipStream_t st) {
    VX_REQUIRE(temperature > 0.f, "sample: temperature must be > 0");
    VX_REQUIRE(vocab > 0 && vocab <= (int64_t)kMaxChunks * kSmChunk, "sample: vocab must be 1..262144");
    const int nch = (int)vx_cdiv(vocab, kSmChunk);
    const size_t need = stochastic_workspace_bytes(rows, vocab);
    if (!ws) {
        VX_TRY(stream_workspace(st, need, &ws));
    } else if (ws_bytes < need) {
        return set_error("sample: workspace too small");
    }
    StochLayout L;
    stoch_layout(ws, rows, rows, nch, &L);
    const float inv_t = 1.0f / temperature;
    stats(logits, ldt, rows, vocab, inv_t, L.cm, L.cz, nch, st);
    DrawArgs a{logits, nullptr, uni, ustride, L.cm, L.cz, nch, vocab, inv_t, L.desc, L.ss, L.cs, L.lastpos,
               out, next_ids, next_stride};
    launch_draws<true>(a, ldt, rows, st);
    VX_HIP(hipGetLastError());
    return 0;
}

int stochastic_accept_launch(const void *tl, const void *dl, int ldt, const uint32_t *cand,
                             const float *uni, int32_t *accepted, uint32_t *tokens, int64_t batch,
                             int64_t k, int64_t vocab, float temperature, bool draft_step_major, void *ws,
                             size_t ws_bytes, hipStream_t st) {
    VX_REQUIRE(temperature > 0.f, "accept_stochastic: temperature must be > 0");
    VX_REQUIRE(k >= 1, "accept_stochastic: k must be >= 1");
    VX_REQUIRE(vocab > 0 && vocab <= (int64_t)kMaxChunks * kSmChunk, "accept_stochastic: vocab must be 1..262144");
    const int nch = (int)vx_cdiv(vocab, kSmChunk);
    const int64_t trows = batch * (k + 1), drows = batch * k;
    const size_t need = stochastic_workspace_bytes(trows + drows, vocab);
    if (!ws) {
        VX_TRY(stream_workspace(st, need, &ws));
    } else if (ws_bytes < need) {
        return set_error("accept_stochastic: workspace too small");
    }
    StochLayout L;
    stoch_layout(ws, trows + drows, batch, nch, &L);
    float *cm_d = L.cm + trows * nch, *cz_d = L.cz + trows * nch;
    const float inv_t = 1.0f / temperature;
    stats(tl, ldt, trows, vocab, inv_t, L.cm, L.cz, nch, st);
    stats(dl, ldt, drows, vocab, inv_t, cm_d, cz_d, nch, st);
    hipLaunchKernelGGL(stochastic_walk_kernel, dim3((unsigned)vx_cdiv(batch, 64)), dim3(64), 0, st, tl, dl, ldt,
                       cand, uni, L.cm, L.cz, cm_d, cz_d, nch, vocab, (int)k, batch, (int)draft_step_major, inv_t,
                       accepted, tokens, L.desc);
    DrawArgs a{tl, dl, nullptr, 0, nullptr, nullptr, nch, vocab, inv_t, L.desc, L.ss, L.cs, L.lastpos,
               tokens, nullptr, 0};
    launch_draws<false>(a, ldt, batch, st);
    VX_HIP(hipGetLastError());
    return 0;
}

// ---- engine helpers --------------------------------------------------------
int rmsnorm_launch(const uint16_t *x, const uint16_t *w, uint16_t *y, const uint32_t *row_idx,
                   int64_t rows, int64_t H, float eps, int out_dt, hipStream_t st) {
    if (H % 8 != 0 || H > 8 * 1024) return set_error("rmsnorm: hidden size must be a multiple of 8 and <= 8192");
    if (rows == 0) return 0;
    const unsigned threads = (unsigned)vx_cdiv(H / 8, 64) * 64;
    hipLaunchKernelGGL(rmsnorm_bf16_kernel, dim3((unsigned)rows), dim3(threads), 0, st, x, w, y, row_idx, (int)H,
                       eps, out_dt, INT64_MAX, (uint16_t *)nullptr, (int64_t)1);
    VX_HIP(hipGetLastError());
    return 0;
}

// Embedding lookup fused with the first layer's norm: h[r] = embed[ids[r *
// ids_stride]] (ids clamped to the vocabulary) and y[r] = RMSNorm(h[r]) * w.
int embed_rmsnorm_launch(const uint32_t *ids, int64_t ids_stride, const uint16_t *embed, int64_t vocab,
                         const uint16_t *w, uint16_t *h, uint16_t *y, int64_t rows, int64_t H, float eps, int out_dt,
                         hipStream_t st) {
    if (H % 8 != 0 || H > 8 * 1024) return set_error("rmsnorm: hidden size must be a multiple of 8 and <= 8192");
    if (vocab < 1) return set_error("embedding: empty vocabulary");
    if (rows == 0) return 0;
    const unsigned threads = (unsigned)vx_cdiv(H / 8, 64) * 64;
    hipLaunchKernelGGL(rmsnorm_bf16_kernel, dim3((unsigned)rows), dim3(threads), 0, st, embed, w, y, ids, (int)H,
                       eps, out_dt, vocab, h, ids_stride);
    VX_HIP(hipGetLastError());
    return 0;
}

int qk_rope_scatter_launch(const uint16_t *qkv, const uint16_t *qn, const uint16_t *kn,
                           const uint16_t *cos_t, const uint16_t *sin_t, const uint32_t *pos,
                           const uint32_t *pages, const uint32_t *slots, uint16_t *qout,
                           uint16_t *kp, uint16_t *vp, int64_t rows, int HQ, int HK, int D, int ps,
                           float eps, int kv_dt, hipStream_t st) {
    if (D > 256 || D % 2 != 0) return set_error("qk_rope_scatter: head_dim must be even and <= 256");
    if (rows == 0) return 0;
    const int64_t waves = rows * (HQ + 2 * HK);
    hipLaunchKernelGGL(qk_rope_scatter_kernel<false>, dim3((unsigned)vx_cdiv(waves, 4)), dim3(256), 0, st, qkv,
                       nullptr, 0, qn, kn, cos_t, sin_t, pos, pages, slots, qout, kp, vp, (int)rows, HQ, HK, D,
                       ps, eps, kv_dt);
    VX_HIP(hipGetLastError());
    return 0;
}

// q/k norm + RoPE + KV write straight from the qkv projection's split partials.
int qkv_partial_rope_scatter_launch(const float *partial, int splits, const uint16_t *qn, const uint16_t *kn,
                                    const uint16_t *cos_t, const uint16_t *sin_t, const uint32_t *pos,
                                    const uint32_t *pages, const uint32_t *slots, uint16_t *qout, uint16_t *kp,
                                    uint16_t *vp, int64_t rows, int HQ, int HK, int D, int ps, float eps, int kv_dt,
                                    hipStream_t st) {
    if (D > 256 || D % 2 != 0) return set_error("qk_rope_scatter: head_dim must be even and <= 256");
    if (splits < 1 || splits > kMaxFusedSplits) return set_error("qk_rope_scatter: split count out of range");
    if (rows == 0) return 0;
    const int64_t waves = rows * (HQ + 2 * HK);
    hipLaunchKernelGGL(qk_rope_scatter_kernel<true>, dim3((unsigned)vx_cdiv(waves, 4)), dim3(256), 0, st, nullptr,
                       partial, splits, qn, kn, cos_t, sin_t, pos, pages, slots, qout, kp, vp, (int)rows, HQ, HK,
                       D, ps, eps, kv_dt);
    VX_HIP(hipGetLastError());
    return 0;
}

// h += finish(partials) (bf16 residual), then y = RMSNorm(h) * ln when ln != null.
int residual_rmsnorm_launch(const float *partial, int splits, float acc_scale, uint16_t *h, const uint16_t *ln,
                            uint16_t *y, int64_t rows, int64_t H, float eps, int out_dt, hipStream_t st) {
    if (H % 8 != 0 || H > 8 * 1024) return set_error("rmsnorm: hidden size must be a multiple of 8 and <= 8192");
    if (splits < 1 || splits > kMaxFusedSplits) return set_error("residual_rmsnorm: split count out of range");
    if (rows == 0) return 0;
    const unsigned threads = (unsigned)vx_cdiv(H / 8, 64) * 64;
    hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3((unsigned)rows), dim3(threads), 0, st, partial, splits,
                       acc_scale, h, ln, y, (int)rows, (int)H, eps, out_dt);
    VX_HIP(hipGetLastError());
    return 0;
}

}  // namespace vx

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" int vx_rope_inplace(void *x, const void *cos_t, const void *sin_t, const uint32_t *offsets,
                               int64_t n, int64_t h, int64_t d, int64_t max_pos, int dtype,
                               void *stream) {
    VX_REQUIRE(d % 2 == 0, "batched_rope_decode: D must be even");
    VX_REQUIRE(max_pos > 0, "batched_rope_decode: empty tables");
    const int64_t tot = n * h * (d / 2);
    if (tot == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(x && cos_t && sin_t && offsets, "batched_rope_decode: null tensor");
    hipStream_t st = (hipStream_t)stream;
    dim3 grid((unsigned)vx_cdiv(tot, 256));
    if (dtype == VX_F32)
        hipLaunchKernelGGL(rope_kernel<VX_F32>, grid, dim3(256), 0, st, x, cos_t, sin_t, offsets, n, h, d / 2);
    else if (dtype == VX_F16)
        hipLaunchKernelGGL(rope_kernel<VX_F16>, grid, dim3(256), 0, st, x, cos_t, sin_t, offsets, n, h, d / 2);
    else if (dtype == VX_BF16)
        hipLaunchKernelGGL(rope_kernel<VX_BF16>, grid, dim3(256), 0, st, x, cos_t, sin_t, offsets, n, h, d / 2);
    else
        return set_error("batched_rope_decode: unsupported dtype");
    VX_HIP(hipGetLastError());
    return 0;
}

extern "C" int vx_kv_scatter(void *pool, const void *values, const uint32_t *page_ids,
                             const uint32_t *slots, int64_t n, int64_t num_pages, int64_t h,
                             int64_t page_size, int64_t d, int dtype, void *stream) {
    VX_REQUIRE(dtype == VX_F32 || dtype == VX_F16 || dtype == VX_BF16, "batched_scatter: unsupported dtype");
    const int64_t esz = dtype == VX_F32 ? 4 : 2;
    VX_REQUIRE((d * esz) % 4 == 0, "batched_scatter: row bytes must be a multiple of 4");
    if (n == 0 || h == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(pool && values && page_ids && slots, "batched_scatter: null tensor");
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(scatter_kernel, dim3((unsigned)(n * h)), dim3(64), 0, st, (uint8_t *)pool,
                       (const uint8_t *)values, page_ids, slots, n, h, page_size, d * esz, num_pages);
    VX_HIP(hipGetLastError());
    return 0;
}

extern "C" int vx_argmax_rows(const void *logits, uint32_t *out, int64_t rows, int64_t vocab,
                              int logits_dtype, void *stream) {
    if (rows == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(logits && out, "argmax: null tensor");
    return argmax_accept_launch(logits, logits_dtype, rows, vocab, 0, 1, nullptr, 0, nullptr, nullptr,
                                nullptr, nullptr, out, nullptr, 0, nullptr, 0, (hipStream_t)stream);
}

extern "C" int vx_accept_greedy(const void *logits, const uint32_t *candidates, int32_t *accepted,
                                uint32_t *tokens, int64_t batch, int64_t k, int64_t vocab,
                                int logits_dtype, void *stream) {
    VX_REQUIRE(k >= 1, "draft_k must be >= 1");
    VX_REQUIRE(k + 1 <= 64, "accept_greedy: k too large");
    if (batch == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(logits && candidates && accepted && tokens, "accept_greedy: null tensor");
    return argmax_accept_launch(logits, logits_dtype, batch * (k + 1), vocab, 1, (int)(k + 1), candidates,
                                (int)k, accepted, tokens, nullptr, nullptr, nullptr, nullptr, 0, nullptr,
                                0, (hipStream_t)stream);
}

extern "C" int vx_accept_tree(const void *logits, const int32_t *parents, const uint32_t *node_tokens,
                              int32_t *accepted, int32_t *path, uint32_t *tokens, int64_t batch,
                              int64_t r, int64_t vocab, int logits_dtype, void *stream) {
    VX_TRY(check_tree_parents(parents, r, "accept_tree"));
    if (batch == 0) return 0;
    return argmax_accept_launch(logits, logits_dtype, batch * r, vocab, 2, (int)r, node_tokens, 0, accepted,
                                tokens, path, parents, nullptr, nullptr, 0, nullptr, 0, (hipStream_t)stream);
}

extern "C" int vx_accept_stochastic(const void *target_logits, const void *draft_logits,
                                    const uint32_t *candidates, const float *uniforms, int32_t *accepted,
                                    uint32_t *tokens, int64_t batch, int64_t k, int64_t vocab,
                                    float temperature, int logits_dtype, void *workspace,
                                    size_t workspace_bytes, void *stream) {
    if (batch == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(target_logits && draft_logits && candidates && uniforms && accepted && tokens,
               "accept_stochastic: null tensor");
    return stochastic_accept_launch(target_logits, draft_logits, logits_dtype, candidates, uniforms, accepted,
                                    tokens, batch, k, vocab, temperature, false, workspace, workspace_bytes,
                                    (hipStream_t)stream);
}

extern "C" int vx_sample_rows(const void *logits, const float *uniforms, int64_t uniform_stride,
                              uint32_t *out, int64_t rows, int64_t vocab, float temperature,
                              int logits_dtype, void *workspace, size_t workspace_bytes, void *stream) {
    if (rows == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(logits && uniforms && out, "sample: null tensor");
    return sample_rows_launch(logits, logits_dtype, uniforms, uniform_stride, out, rows, vocab, temperature,
                              nullptr, 0, workspace, workspace_bytes, (hipStream_t)stream);
}
