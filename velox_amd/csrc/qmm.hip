// int4 g64 affine GEMM for the verify rows (M = k+1 per sequence, M = 5..80
// and beyond), gfx950.
//
// Replaces qmm_4bit (reference src/paged/metal_kernels.rs:2069-2309, naive MSL
// :418-479).  Math: y[m,n] = sum_k x[m,k] * (q[n,k] * s[n,g] + b[n,g]).
//
// Fast path (X in f16, scales/biases in f16, group 64, K % 256 == 0):
//   * workgroup = 4 waves; a wave owns NT column tiles of 16 and MT row tiles
//     of 16 (v_mfma_f32_16x16x32_f16, f32 accumulation);
//   * each lane reads 8 bytes (16 nibbles) of one weight row per group; the
//     nibbles become f16 with the magic-exponent trick ((q | 0x6400) = 1024+q)
//     and are dequantised with one v_pk_add_f16 + one v_pk_fma_f16 per pair,
//     so w = fma_f16(q, s, b) carries a single rounding;
//   * the activation block for 4 groups is staged once per workgroup in LDS in
//     MFMA fragment order (one ds_read_b128 per fragment), permuted to match
//     the nibble pairing (k, k+4) of the dequantised registers;
//   * split-K over groups when the column grid alone cannot fill the 256 CUs:
//     partial tiles go to a workspace and a second, element-parallel kernel
//     sums them in split order (deterministic) and applies the epilogue.  No
//     workgroup waits on another: a device-scope fence on gfx950 writes back
//     the XCD's whole L2, which made an in-kernel "last workgroup reduces"
//     handshake far slower than the extra launch;
//   * work items are laid out so consecutive items land on the same XCD
//     (dispatch is round-robin over the 8 XCDs), keeping the splits of one
//     column block inside one L2.
// bf16 activations (the reference's bf16 qmm contract) use the same tiling
// with exact integer codes as the B operand (bf16 128+q) and the group scale
// applied per group: y += s*sum(x*q) + b*sum(x).
// Everything else (f32, other group sizes, unaligned shapes) goes to a plain
// one-thread-per-output kernel with the reference's arithmetic.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <map>
#include <mutex>
#include <string>
#include <type_traits>

#include "vx_common.h"

namespace vx {

namespace {

constexpr int kWaves = 4;
constexpr int kChunkGroups = 4;          // groups of 64 staged per LDS chunk
constexpr size_t kCounterBytes = 65536;  // reserved head of the workspace (kept zero)
constexpr size_t kMaxPartialBytes = (size_t)96 << 20;
// Packed weight layout (the engine's): per 32-row tile and 128-wide k step one
// block of kPackBlock bytes, tiles contiguous over their steps so a wave
// streams contiguous memory.  Lane L of a v_mfma_f32_32x32x16 B operand holds
// row L%32 of the tile and, for MFMA j (j < 8) of the step, the 8 k values
// 16j + 8*(L/32) .. +7: one word, with the nibbles of k0..k7 at positions
// 0,4,1,5,2,6,3,7 (the order dequant8 emits).  Bytes [0, 1024): words 0..3 of
// every lane (16 bytes at 16 L); [1024, 2048): words 4..7; [2048, 2304): per
// row r, at 2048 + 8r, (scale, bias) of the step's two groups as f16
// (s0, b0, s1, b1).  Words 0..3 belong to the first group, 4..7 to the second.
constexpr int kPackBlock = 2304;
// Internal epilogue: raw f32 split partials [splits][M][N] (also for one
// split); the consumer kernel reduces them in split order and finishes.
constexpr int kEpiPartial = 100;
constexpr int kMaxPartialSplits = 8;  // what the fused consumers read

struct QmmArgs {
    const void *x;
    const uint32_t *w;
    const uint16_t *s;
    const uint16_t *b;
    void *y;
    const void *resid;
    float *partial;
    int M, N, K, G;
    int splits, gps;
    int S, sps;  // streaming kernel: 128-wide k steps, steps per split
    int col_blocks, m_blocks, per_xcd, total_items;
    int epi, round_dt, y_dt;
    float acc_scale;    // 2^x_shift
    float store_scale;  // 2^-y_shift
    // STORE epilogue of the packed kernels: optional greedy-argmax partials of
    // the stored values, (value, first index) per (row, 128-column block) at
    // [row * ceil(N/128) + block]; NaN never wins, ties keep the smaller index
    float *amax_v;
    uint32_t *amax_i;
    // optional per-column bias [N] in y_dt, added to the f32 accumulator
    // before its single rounding (STORE, metal_kernels.rs:473-474)
    const void *bias;
};

typedef unsigned short ushort8 __attribute__((ext_vector_type(8)));

// [0..7] -> [0,4,1,5,2,6,3,7]: element e of a fragment holds k = perm(e), the
// order in which the dequantised nibble pairs (k, k+4) land in registers.
__device__ __forceinline__ uint4 permute_k8(uint4 v) {
    // halves: v.x = (h0,h1) v.y = (h2,h3) v.z = (h4,h5) v.w = (h6,h7)
    uint4 o;
    o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);  // (h0, h4)
    o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);  // (h1, h5)
    o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);  // (h2, h6)
    o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);  // (h3, h7)
    return o;
}

__device__ __forceinline__ half8_t dequant_f16(uint32_t word, half2_t s2, half2_t b2) {
    const half2_t off = {(vx_half)1024.0f, (vx_half)1024.0f};
    half8_t r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t bits = ((word >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
        half2_t q = __builtin_bit_cast(half2_t, bits) - off;
        half2_t w = q * s2 + b2;
        r[2 * j] = w[0];
        r[2 * j + 1] = w[1];
    }
    return r;
}

// v_and_or_b32 with both constants in VGPRs (CDNA3 VOP3 takes no literal,
// so the compiler otherwise splits it into v_and + v_or).
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t bits) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "v"(mask), "v"(bits));
    return r;
}

// Constants of dequant8, kept in VGPRs by the caller.
struct DqConst {
    uint32_t m_lo, m_hi, magic_lo, magic_hi;
    half2_t off_lo, off_hi;
};
__device__ __forceinline__ DqConst dq_const() {
    DqConst c;
    c.m_lo = 0x000F000Fu;
    c.m_hi = 0x00F000F0u;
    c.magic_lo = 0x64006400u;  // f16 1024: nibble at mantissa bits 0-3 reads as 1024 + q
    c.magic_hi = 0x54005400u;  // f16 64: nibble at mantissa bits 4-7 reads as 64 + q
    c.off_lo = (half2_t){(vx_half)1024.0f, (vx_half)1024.0f};
    c.off_hi = (half2_t){(vx_half)64.0f, (vx_half)64.0f};
    return c;
}

// Eight nibbles of one word -> eight f16 weights fma(q, s, b) (one rounding),
// in the order (n0, n4, n1, n5, n2, n6, n3, n7): pairs (n_j, n_j+4) share a
// register.  Nibbles at bits 0-3 / 4-7 of each half are read in place with
// exponent 1024 / 64; the upper byte pair after one shift: 13 VALU per word.
__device__ __forceinline__ half8_t dequant8(uint32_t word, half2_t s2, half2_t b2, const DqConst &c) {
    const uint32_t w8 = word >> 8;
    const half2_t p0 = __builtin_bit_cast(half2_t, and_or(word, c.m_lo, c.magic_lo)) - c.off_lo;
    const half2_t p1 = __builtin_bit_cast(half2_t, and_or(word, c.m_hi, c.magic_hi)) - c.off_hi;
    const half2_t p2 = __builtin_bit_cast(half2_t, and_or(w8, c.m_lo, c.magic_lo)) - c.off_lo;
    const half2_t p3 = __builtin_bit_cast(half2_t, and_or(w8, c.m_hi, c.magic_hi)) - c.off_hi;
    const half2_t w0 = p0 * s2 + b2, w1 = p1 * s2 + b2, w2 = p2 * s2 + b2, w3 = p3 * s2 + b2;
    return (half8_t){w0[0], w0[1], w1[0], w1[1], w2[0], w2[1], w3[0], w3[1]};
}

__device__ __forceinline__ bf16x8_t codes_bf16(uint32_t word) {
    ushort8 r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t bits = ((word >> (4 * j)) & 0x000F000Fu) | 0x43004300u;
        r[2 * j] = (unsigned short)(bits & 0xffffu);
        r[2 * j + 1] = (unsigned short)(bits >> 16);
    }
    return __builtin_bit_cast(bf16x8_t, r);
}

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + __expf(-v)); }

__device__ __forceinline__ float round_dt(float v, int dt) {
    if (dt == VX_BF16) return round_to<VX_BF16>(v);
    if (dt == VX_F16) return round_to<VX_F16>(v);
    return v;
}
__device__ __forceinline__ void store_dt(void *p, int64_t i, float v, int dt) {
    if (dt == VX_BF16)
        st_elem<VX_BF16>(p, i, v);
    else if (dt == VX_F16)
        st_elem<VX_F16>(p, i, v);
    else
        st_elem<VX_F32>(p, i, v);
}
__device__ __forceinline__ float load_dt(const void *p, int64_t i, int dt) {
    if (dt == VX_BF16) return ld_elem<VX_BF16>(p, i);
    if (dt == VX_F16) return ld_elem<VX_F16>(p, i);
    return ld_elem<VX_F32>(p, i);
}

// Epilogue of one output element (STORE / RESIDUAL).
__device__ __forceinline__ void epi_elem(const QmmArgs &a, int row, int col, float acc) {
    const int64_t idx = (int64_t)row * a.N + col;
    float v = acc * a.acc_scale;
    if (a.bias) v += load_dt(a.bias, col, a.y_dt);
    v = round_dt(v, a.round_dt);
    if (a.epi == VX_EPI_RESIDUAL) v = round_dt(load_dt(a.resid, idx, a.y_dt) + v, a.round_dt);
    store_dt(a.y, idx, v * a.store_scale, a.y_dt);
}

// SwiGLU epilogue of one (row, feature) from its gate and up accumulators.
__device__ __forceinline__ void epi_swiglu(const QmmArgs &a, int row, int f, float gacc, float uacc) {
    const float g = round_dt(gacc * a.acc_scale, a.round_dt);
    const float u = round_dt(uacc * a.acc_scale, a.round_dt);
    const float v = round_dt(round_dt(silu_f(g), a.round_dt) * u, a.round_dt);
    store_dt(a.y, (int64_t)row * (a.N / 2) + f, v * a.store_scale, a.y_dt);
}

// Writes a wave's accumulators: the split-K partial tile when the K range is
// split (qmm_reduce_kernel finishes), else the epilogue.  C fragment layout of
// v_mfma_f32_16x16x32: lane holds column lane%16, rows 4*(lane/16) + r.
template <int MT, int NT>
__device__ __forceinline__ void store_acc(const QmmArgs &a, const floatx4 (&acc)[MT][NT], int m0, int col0,
                                          int sp, int kq) {
    if (a.splits > 1 || a.epi == kEpiPartial) {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int col = col0 + nt * 16;
                if (col >= a.N) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = m0 + t * 16 + 4 * kq + r;
                    if (row < a.M) a.partial[((int64_t)sp * a.M + row) * a.N + col] = acc[t][nt][r];
                }
            }
        return;
    }
    if (a.epi == VX_EPI_SWIGLU) {
        // tiles come in (gate, up) pairs: global tile 2f = gate rows, 2f+1 = up rows
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int nt = 0; nt + 1 < NT; nt += 2) {
                const int gtile = (col0 - (col0 & 15)) / 16 + nt;
                const int f = (gtile / 2) * 16 + (col0 & 15);
                if (col0 + nt * 16 >= a.N) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = m0 + t * 16 + 4 * kq + r;
                    if (row < a.M) epi_swiglu(a, row, f, acc[t][nt][r], acc[t][nt + 1][r]);
                }
            }
        return;
    }
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int col = col0 + nt * 16;
            if (col >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = m0 + t * 16 + 4 * kq + r;
                if (row < a.M) epi_elem(a, row, col, acc[t][nt][r]);
            }
        }
}

template <int MT, int NT, bool XBF>
__global__ __launch_bounds__(256) void qmm_int4_kernel(QmmArgs a) {
    // X tile of one chunk (4 groups x 64 k) in MFMA fragment order, double buffered
    constexpr int UNITS = kChunkGroups * 2 * MT * 64;  // 16-byte fragments per chunk
    constexpr int UPT = UNITS / 256;                   // per thread (= 2 * MT)
    __shared__ uint4 xs[2][UNITS];
    __shared__ float xsum[XBF ? 2 : 1][XBF ? kChunkGroups * MT * 16 : 1];

    const int bid = blockIdx.x;
    const int item = (bid & 7) * a.per_xcd + (bid >> 3);
    if (item >= a.total_items) return;
    const int cb = item / a.splits;
    const int sp = item - cb * a.splits;
    const int m0 = blockIdx.y * MT * 16;
    const int g_lo = sp * a.gps;
    const int g_hi = min(a.G, g_lo + a.gps);  // g_lo, g_hi are multiples of 4
    const int nchunks = (g_hi - g_lo) / kChunkGroups;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kq = lane >> 4;
    const int col0 = cb * (kWaves * NT * 16) + wave * NT * 16 + (lane & 15);
    const int kw = a.K / 8;

    // per-thread staging map: unit u = tid + 256 j -> (row, k offset within the chunk)
    const uint16_t *xh = (const uint16_t *)a.x;
    int xoff[UPT];
    bool xok[UPT];
#pragma unroll
    for (int j = 0; j < UPT; j++) {
        const int r = wave + 4 * j;
        const int t = r % MT;
        const int q = r / MT;
        const int row = m0 + t * 16 + (lane & 15);
        xok[j] = row < a.M;
        xoff[j] = (xok[j] ? row : 0) * a.K + (q >> 1) * 64 + 8 * (2 * kq + (q & 1));
    }
    const uint32_t *wbase[NT];
    const uint16_t *sbase[NT], *bbase[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int col = min(col0 + nt * 16, a.N - 1);
        wbase[nt] = a.w + (int64_t)col * kw + 2 * kq;
        sbase[nt] = a.s + (int64_t)col * a.G;
        bbase[nt] = a.b + (int64_t)col * a.G;
    }

    floatx4 acc[MT][NT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[t][nt] = (floatx4){0.f, 0.f, 0.f, 0.f};

    uint2 wc[kChunkGroups][NT], sc[NT], bc[NT];  // current chunk weights / affine params
    uint4 xr[UPT];                              // next chunk activations (registers)

    auto load_w = [&](int g, uint2 (&w)[kChunkGroups][NT], uint2 (&sv)[NT], uint2 (&bv)[NT]) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int gg = 0; gg < kChunkGroups; gg++) w[gg][nt] = *(const uint2 *)(wbase[nt] + (g + gg) * 8);
            sv[nt] = *(const uint2 *)(sbase[nt] + g);
            bv[nt] = *(const uint2 *)(bbase[nt] + g);
        }
    };
    auto load_x = [&](int g) {
#pragma unroll
        for (int j = 0; j < UPT; j++)
            xr[j] = xok[j] ? *(const uint4 *)(xh + xoff[j] + g * 64) : make_uint4(0u, 0u, 0u, 0u);
    };
    auto store_x = [&](int buf, int g) {
#pragma unroll
        for (int j = 0; j < UPT; j++) xs[buf][tid + 256 * j] = permute_k8(xr[j]);
        if constexpr (XBF) {
            for (int idx = tid; idx < kChunkGroups * MT * 16; idx += 256) {
                const int gg = idx / (MT * 16);
                const int rr = idx - gg * MT * 16;
                float sum = 0.f;
                if (m0 + rr < a.M) {
                    const uint16_t *xrow = xh + (int64_t)(m0 + rr) * a.K + (g + gg) * 64;
                    for (int e = 0; e < 64; e++) sum += bf16_bits_to_f32(xrow[e]);
                }
                xsum[buf][idx] = sum;
            }
        }
    };

    load_w(g_lo, wc, sc, bc);
    load_x(g_lo);
    store_x(0, g_lo);
    __syncthreads();

    for (int c = 0; c < nchunks; c++) {
        const int buf = c & 1;
        const bool more = c + 1 < nchunks;
        const int gn = g_lo + (c + 1) * kChunkGroups;
        uint2 wn[kChunkGroups][NT], sn[NT], bn[NT];
        if (more) {
            load_x(gn);
            load_w(gn, wn, sn, bn);
        }
#pragma unroll
        for (int gg = 0; gg < kChunkGroups; gg++) {
            if constexpr (!XBF) {
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    half8_t af[MT];
#pragma unroll
                    for (int t = 0; t < MT; t++)
                        af[t] = __builtin_bit_cast(half8_t, xs[buf][((gg * 2 + s) * MT + t) * 64 + lane]);
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        const uint32_t word = s == 0 ? wc[gg][nt].x : wc[gg][nt].y;
                        const uint32_t sbits = gg < 2 ? sc[nt].x : sc[nt].y;
                        const uint32_t bbits = gg < 2 ? bc[nt].x : bc[nt].y;
                        const uint16_t sh = (gg & 1) ? (uint16_t)(sbits >> 16) : (uint16_t)sbits;
                        const uint16_t bh = (gg & 1) ? (uint16_t)(bbits >> 16) : (uint16_t)bbits;
                        const vx_half svh = __builtin_bit_cast(vx_half, sh);
                        const vx_half bvh = __builtin_bit_cast(vx_half, bh);
                        const half8_t bf = dequant_f16(word, (half2_t){svh, svh}, (half2_t){bvh, bvh});
#pragma unroll
                        for (int t = 0; t < MT; t++)
                            acc[t][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], bf, acc[t][nt], 0, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const uint32_t sbits = gg < 2 ? sc[nt].x : sc[nt].y;
                    const uint32_t bbits = gg < 2 ? bc[nt].x : bc[nt].y;
                    const float svf = bf16_bits_to_f32((gg & 1) ? (uint16_t)(sbits >> 16) : (uint16_t)sbits);
                    const float bvf = bf16_bits_to_f32((gg & 1) ? (uint16_t)(bbits >> 16) : (uint16_t)bbits);
                    const float boff = bvf - 128.0f * svf;
                    const bf16x8_t b0 = codes_bf16(wc[gg][nt].x);
                    const bf16x8_t b1 = codes_bf16(wc[gg][nt].y);
#pragma unroll
                    for (int t = 0; t < MT; t++) {
                        floatx4 tmp = {0.f, 0.f, 0.f, 0.f};
                        tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8_t, xs[buf][((gg * 2 + 0) * MT + t) * 64 + lane]), b0, tmp, 0, 0, 0);
                        tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8_t, xs[buf][((gg * 2 + 1) * MT + t) * 64 + lane]), b1, tmp, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const float xsr = xsum[buf][gg * MT * 16 + t * 16 + 4 * kq + r];
                            acc[t][nt][r] += svf * tmp[r] + boff * xsr;
                        }
                    }
                }
            }
        }
        if (more) {
            store_x(buf ^ 1, gn);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
#pragma unroll
                for (int gg = 0; gg < kChunkGroups; gg++) wc[gg][nt] = wn[gg][nt];
                sc[nt] = sn[nt];
                bc[nt] = bn[nt];
            }
        }
        __syncthreads();
    }

    store_acc<MT, NT>(a, acc, m0, col0, sp, kq);
}

// f16 streaming kernel (the verify path's GEMM).  K advances in steps of 128
// (two groups).  In a step, lane L reads one 16-byte piece of weight row
// col = L%16 (+16 nt): the 32 k values 32*(L/16) .. +31, four packed words.
// MFMA j (j < 4) of the step takes word j from every lane, so its 32-wide k
// set is {32*kq + 8j + e}; the activation fragments are staged in LDS with the
// same k set per lane (16 contiguous bytes, then permute_k8), so the dot
// product is unchanged.  A lane's group is 2*step + kq/2, so each lane
// dequantises with its own scale/bias.
// Software pipeline: the weights, scales and activations of step s+P are
// requested before step s is computed, in a ring of P+1 register slots (the
// step loop is unrolled by the ring size so every slot is a fixed register
// set); the activations of step s+1 move to the other LDS buffer after the
// MFMAs of step s, one barrier per step.
template <int MT, int NT, int P>
__global__ __launch_bounds__(256) void qmm_f16_stream_kernel(QmmArgs a) {
    constexpr int R = P + 1;
    static_assert(R >= 2 && R <= 6, "ring of 2..6 slots");
    constexpr int FR = 4 * MT;  // activation fragments (j, t) per step
    constexpr int UPT = MT;     // 16-byte fragment pieces per thread per step (FR * 64 / 256)
    __shared__ uint4 xs[2][FR * 64];

    const int bid = blockIdx.x;
    const int item = (bid & 7) * a.per_xcd + (bid >> 3);
    if (item >= a.total_items) return;
    const int cb = item / a.splits;
    const int sp = item - cb * a.splits;
    const int m0 = blockIdx.y * MT * 16;
    const int s_lo = sp * a.sps;
    const int s_hi = min(a.S, s_lo + a.sps);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kq = lane >> 4;
    const int col0 = cb * (kWaves * NT * 16) + wave * NT * 16 + (lane & 15);

    // activation pieces: unit u = tid + 256 i is fragment (j, t) = divmod(u / 64, MT), lane u % 64;
    // rows past M re-read row M-1 (finite values whose results are never stored)
    const uint16_t *xh = (const uint16_t *)a.x;
    int xoff[UPT];
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + 256 * i;
        const int ln = u & 63;
        const int jt = u >> 6;
        const int j = jt / MT;
        const int t = jt - j * MT;
        const int row = min(m0 + t * 16 + (ln & 15), a.M - 1);
        xoff[i] = row * a.K + 32 * (ln >> 4) + 8 * j;
    }
    // MLX layout: weight row col, words 16 st + 4 kq .. +3; scales/biases
    // [N, G] (the pair of groups of step st is one 32-bit word).
    const uint4 *wrow[NT];
    const uint32_t *srow[NT], *brow[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int col = min(col0 + nt * 16, a.N - 1);
        wrow[nt] = (const uint4 *)(a.w + (int64_t)col * (a.K / 8)) + kq;
        srow[nt] = (const uint32_t *)(a.s + (int64_t)col * a.G);
        brow[nt] = (const uint32_t *)(a.b + (int64_t)col * a.G);
    }
    // byte selector replicating the lane's group half (kq/2) into both halves
    const uint32_t hsel = (kq & 2) ? 0x03020302u : 0x01000100u;
    const DqConst dq = dq_const();

    floatx4 acc[MT][NT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[t][nt] = (floatx4){0.f, 0.f, 0.f, 0.f};

    uint4 wr[R][NT];
    uint32_t sr[R][NT], br[R][NT];
    uint4 xr[R][UPT];

    auto issue = [&](int st, uint4 (&w)[NT], uint32_t (&sv)[NT], uint32_t (&bv)[NT], uint4 (&xv)[UPT]) {
#pragma unroll
        for (int i = 0; i < UPT; i++) xv[i] = *(const uint4 *)(xh + xoff[i] + st * 128);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            w[nt] = wrow[nt][st * 4];
            sv[nt] = srow[nt][st];
            bv[nt] = brow[nt][st];
        }
    };
    // dequant8 emits the word's nibble pairs (k, k+4): permute X to match
    auto stage = [&](int buf, const uint4 (&xv)[UPT]) {
#pragma unroll
        for (int i = 0; i < UPT; i++) xs[buf][tid + 256 * i] = permute_k8(xv[i]);
    };

    // One step: request step st+P into its ring slot (clamped to the last
    // step so every path issues the same loads and the compiler's wait
    // counts stay exact), run the MFMAs of step st, stage the activations of
    // step st+1.
    auto step = [&](int st, auto slot_c) {
        constexpr int I = decltype(slot_c)::value;
        constexpr int NX = (I + P) % R;
        issue(min(st + P, s_hi - 1), wr[NX], sr[NX], br[NX], xr[NX]);
        // keep the prefetch at the head of the step: if the scheduler sinks it
        // below the MFMAs, consuming an older slot waits for every load in flight
        __builtin_amdgcn_sched_barrier(0);
        const int buf = (st - s_lo) & 1;
        half2_t s2[NT], b2[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            s2[nt] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sr[I][nt], sr[I][nt], hsel));
            b2[nt] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(br[I][nt], br[I][nt], hsel));
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            half8_t af[MT];
#pragma unroll
            for (int t = 0; t < MT; t++) af[t] = __builtin_bit_cast(half8_t, xs[buf][(j * MT + t) * 64 + lane]);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const uint32_t word = j == 0 ? wr[I][nt].x : j == 1 ? wr[I][nt].y : j == 2 ? wr[I][nt].z : wr[I][nt].w;
                const half8_t bf = dequant8(word, s2[nt], b2[nt], dq);
#pragma unroll
                for (int t = 0; t < MT; t++)
                    acc[t][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], bf, acc[t][nt], 0, 0, 0);
            }
        }
        stage(buf ^ 1, xr[(I + 1) % R]);  // past the last step this stages a copy nobody reads
        __syncthreads();
    };

#pragma unroll
    for (int i = 0; i < P; i++) issue(min(s_lo + i, s_hi - 1), wr[i], sr[i], br[i], xr[i]);
    stage(0, xr[0]);
    __syncthreads();

    int st = s_lo;
    for (; st + R <= s_hi; st += R) {
        step(st + 0, std::integral_constant<int, 0>{});
        if constexpr (R > 1) step(st + 1, std::integral_constant<int, 1 % R>{});
        if constexpr (R > 2) step(st + 2, std::integral_constant<int, 2 % R>{});
        if constexpr (R > 3) step(st + 3, std::integral_constant<int, 3 % R>{});
        if constexpr (R > 4) step(st + 4, std::integral_constant<int, 4 % R>{});
        if constexpr (R > 5) step(st + 5, std::integral_constant<int, 5 % R>{});
    }
    // tail: fewer than R steps remain; slot of step st + i is i
    if (st < s_hi) step(st, std::integral_constant<int, 0>{});
    if constexpr (R > 2) if (st + 1 < s_hi) step(st + 1, std::integral_constant<int, 1 % R>{});
    if constexpr (R > 3) if (st + 2 < s_hi) step(st + 2, std::integral_constant<int, 2 % R>{});
    if constexpr (R > 4) if (st + 3 < s_hi) step(st + 3, std::integral_constant<int, 3 % R>{});
    if constexpr (R > 5) if (st + 4 < s_hi) step(st + 4, std::integral_constant<int, 4 % R>{});
    store_acc<MT, NT>(a, acc, m0, col0, sp, kq);
}

// Word with nibbles k0..k7 (k at bits 4k) -> nibble positions
// (k0, k2, k4, k6, k1, k3, k5, k7), so dequant8's pairs (p, p+4) come out as
// (k0, k1), (k2, k3), ...: natural k order.
__device__ __forceinline__ uint32_t pack_nibbles(uint32_t w) {
    uint32_t o = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        o |= ((w >> (8 * j)) & 0xFu) << (4 * j);             // k 2j     -> position j
        o |= ((w >> (8 * j + 4)) & 0xFu) << (4 * j + 16);   // k 2j + 1 -> position j + 4
    }
    return o;
}

// MLX [N, K/8] words + [N, K/64] scales/biases -> packed blocks.  One
// workgroup of 64 threads per (tile, step) block; thread L writes lane L's
// two 16-byte pieces, threads < 32 also the scale/bias pairs of row L.
__global__ __launch_bounds__(64) void qmm_pack_kernel(const uint32_t *w, const uint16_t *s, const uint16_t *b,
                                                      uint8_t *out, int N, int K) {
    const int S = K / 128, G = K / 64;
    const int64_t blk = blockIdx.x;
    const int tile = (int)(blk / S), st = (int)(blk - (int64_t)tile * S);
    const int lane = threadIdx.x;
    uint8_t *o = out + blk * kPackBlock;
    const int row = tile * 32 + (lane & 31);
    const int kh = lane >> 5;
    const uint4 *src = (const uint4 *)(w + (int64_t)row * (K / 8) + st * 16);
    const uint4 q0 = src[0], q1 = src[1], q2 = src[2], q3 = src[3];
    const uint32_t words[16] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w,
                                q2.x, q2.y, q2.z, q2.w, q3.x, q3.y, q3.z, q3.w};
    uint32_t pw[8];
#pragma unroll
    for (int j = 0; j < 8; j++) pw[j] = pack_nibbles(words[2 * j + kh]);
    *(uint4 *)(o + lane * 16) = make_uint4(pw[0], pw[1], pw[2], pw[3]);
    *(uint4 *)(o + 1024 + lane * 16) = make_uint4(pw[4], pw[5], pw[6], pw[7]);
    if (lane < 32) {
        const int64_t r = (int64_t)tile * 32 + lane;
        const int g = 2 * st;
        const uint32_t p0 = (uint32_t)s[r * G + g] | ((uint32_t)b[r * G + g] << 16);
        const uint32_t p1 = (uint32_t)s[r * G + g + 1] | ((uint32_t)b[r * G + g + 1] << 16);
        *(uint2 *)(o + 2048 + lane * 8) = make_uint2(p0, p1);
    }
}

// Writes a wave's v_mfma_f32_32x32x16 accumulators (lane L, element i: column
// L%32, row 8*(i/4) + 4*(L/32) + i%4 of the 32x32 tile): split partials when
// the K range is split or the caller asked for them, else the epilogue.
// SwiGLU: a 32-column tile is gate rows [16T, 16T+16) then up rows of the same
// features (weights interleaved in 16-row blocks), so lane L < 16 of each half
// pairs with lane L + 16.
template <int MT, int NT>
__device__ __forceinline__ void store_acc32(const QmmArgs &a, const floatx16 (&acc)[MT][NT], int m0, int col0,
                                            int sp, int lane) {
    const int hr = 4 * (lane >> 5);
    const int c = lane & 31;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            // the accumulators are only read with constant indices here; the
            // per-element work below runs on this copy, so a loop the compiler
            // keeps rolled cannot push the accumulators themselves to scratch
            float v[16], u[16];
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = acc[t][nt][i];
            const int col = col0 + nt * 32;
            if (a.splits > 1 || a.epi == kEpiPartial) {
                if (col >= a.N) continue;
                // rows m0 + 32t + hr + ro, ro = 8*(i/4) + i%4: one 64-bit base per
                // tile, 32-bit row offsets
                const int r0 = m0 + 32 * t + hr;
                float *pb = a.partial + ((int64_t)sp * a.M + r0) * a.N + col;
                const int rem = a.M - r0;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int ro = 8 * (i >> 2) + (i & 3);
                    if (ro < rem) pb[ro * a.N] = v[i];
                }
            } else if (a.epi == VX_EPI_SWIGLU) {
#pragma unroll
                for (int i = 0; i < 16; i++) u[i] = __shfl_down(v[i], 16);
                const int tile = (col0 - c) / 32 + nt;
                const int f = tile * 16 + c;
                if (c >= 16 || tile * 32 >= a.N) continue;
                for (int i = 0; i < 16; i++) {
                    const int row = m0 + 32 * t + 8 * (i >> 2) + hr + (i & 3);
                    if (row < a.M) epi_swiglu(a, row, f, v[i], u[i]);
                }
            } else {
                if (col >= a.N) continue;
                for (int i = 0; i < 16; i++) {
                    const int row = m0 + 32 * t + 8 * (i >> 2) + hr + (i & 3);
                    if (row < a.M) epi_elem(a, row, col, v[i]);
                }
            }
        }
}

// GEMM over packed weights on v_mfma_f32_32x32x16_f16 (the engine's path).
// A workgroup is four waves; a wave owns NT tiles of 32 output columns and
// MT tiles of 32 rows.  K advances in 128-wide steps: per step a lane loads
// two 16-byte weight pieces and one (scale, bias) word pair per tile (the
// eight words feed the step's eight MFMAs), and the workgroup stages the
// step's activations in LDS in A-fragment order (lane L: row L%32, k
// 16j + 8*(L/32) .. +7, 16 contiguous bytes, no permute: the packed nibble
// order already yields natural k).  Weights, scales and activations of step
// s+P are requested before step s computes, in a ring of P+1 register slots
// (fixed slots, unconditional clamped loads, the requests pinned at the head
// of the step so the compiler's wait counts stay exact); one barrier per step.
template <int MT, int NT, int P>
__global__ __launch_bounds__(256) void qmm_f16_p32_kernel(QmmArgs a) {
    constexpr int R = P + 1;
    static_assert(R >= 2 && R <= 6, "ring of 2..6 slots");
    constexpr int FR = 8 * MT;       // activation fragments (j, t) per step
    constexpr int UPT = FR * 64 / 256;  // 16-byte pieces per thread per step
    __shared__ uint4 xs[2][FR * 64];

    const int bid = blockIdx.x;
    const int item = (bid & 7) * a.per_xcd + (bid >> 3);
    if (item >= a.total_items) return;
    const int cb = item / a.splits;
    const int sp = item - cb * a.splits;
    const int m0 = blockIdx.y * MT * 32;
    const int s_lo = sp * a.sps;
    const int s_hi = min(a.S, s_lo + a.sps);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col0 = cb * (kWaves * NT * 32) + wave * NT * 32 + (lane & 31);

    // activation pieces: unit u = tid + 256 i is row u / 16, 16-byte chunk u % 16 of the
    // step's 128 k, so one wave instruction reads four whole 256-byte row segments.  In
    // LDS, chunk c of row r sits at r * 16 + (c ^ (r % 16)): sixteen consecutive lanes
    // then hit sixteen distinct 16-byte bank groups both when a row is stored and when
    // a fragment (32 rows, one chunk) is read.  Rows past M re-read row M-1 (finite
    // values whose results are never stored).
    const uint16_t *xh = (const uint16_t *)a.x;
    int xoff[UPT];
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + 256 * i;
        const int row = min(m0 + (u >> 4), a.M - 1);
        xoff[i] = row * a.K + 8 * (u & 15);
    }
    const int xst = (tid >> 4) * 16 + ((tid & 15) ^ ((tid >> 4) & 15));  // + 256 i for piece i
    const int xrd = (lane & 31) * 16;                                     // + 512 t + (2 j ^ xsw)
    const int xsw = (lane >> 5) ^ (lane & 15);
    const uint8_t *wblk[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int tile = min(col0 / 32 + nt, a.N / 32 - 1);
        wblk[nt] = (const uint8_t *)a.w + (int64_t)tile * a.S * kPackBlock;
    }
    constexpr uint32_t kLoHalf = 0x01000100u, kHiHalf = 0x03020302u;
    const DqConst dq = dq_const();

    floatx16 acc[MT][NT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[t][nt][i] = 0.f;

    uint4 wlo[R][NT], whi[R][NT];  // words 0..3 / 4..7 of each tile
    uint2 sr[R][NT];
    uint4 xr[R][UPT];

    auto issue = [&](int st, uint4 (&w0)[NT], uint4 (&w1)[NT], uint2 (&sv)[NT], uint4 (&xv)[UPT]) {
#pragma unroll
        for (int i = 0; i < UPT; i++) xv[i] = *(const uint4 *)(xh + xoff[i] + st * 128);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const uint8_t *bp = wblk[nt] + (int64_t)st * kPackBlock;
            w0[nt] = *(const uint4 *)(bp + lane * 16);
            w1[nt] = *(const uint4 *)(bp + 1024 + lane * 16);
            sv[nt] = *(const uint2 *)(bp + 2048 + (lane & 31) * 8);
        }
    };
    // component-wise copy: a whole-struct copy becomes a memcpy that keeps the
    // register ring in scratch memory
    auto stage = [&](int buf, const uint4 (&xv)[UPT]) {
#pragma unroll
        for (int i = 0; i < UPT; i++) xs[buf][xst + 256 * i] = make_uint4(xv[i].x, xv[i].y, xv[i].z, xv[i].w);
    };
    auto step = [&](int st, auto slot_c) {
        constexpr int I = decltype(slot_c)::value;
        constexpr int NX = (I + P) % R;
        issue(min(st + P, s_hi - 1), wlo[NX], whi[NX], sr[NX], xr[NX]);
        // keep the prefetch at the head of the step: if the scheduler sinks it
        // below the MFMAs, consuming an older slot waits for every load in flight
        __builtin_amdgcn_sched_barrier(0);
        const int buf = (st - s_lo) & 1;
        half2_t s2[NT][2], b2[NT][2];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            s2[nt][0] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sr[I][nt].x, sr[I][nt].x, kLoHalf));
            b2[nt][0] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sr[I][nt].x, sr[I][nt].x, kHiHalf));
            s2[nt][1] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sr[I][nt].y, sr[I][nt].y, kLoHalf));
            b2[nt][1] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sr[I][nt].y, sr[I][nt].y, kHiHalf));
        }
        // sub-step j+1's A fragments are read from LDS before the MFMAs of
        // sub-step j are issued (a scheduling barrier keeps the compiler from
        // sinking the reads next to their use), so the MFMAs cover the LDS
        // latency; the dequant of j+1 interleaves with those MFMAs
        half8_t af[2][MT], bq[2][NT];
        auto lds_a = [&](int j, int c) {
#pragma unroll
            for (int t = 0; t < MT; t++) af[c][t] = __builtin_bit_cast(half8_t, xs[buf][xrd + 512 * t + ((2 * j) ^ xsw)]);
        };
        auto deq_b = [&](int j, int c) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const uint4 q = (j >> 2) ? whi[I][nt] : wlo[I][nt];
                const uint32_t word = (j & 3) == 0 ? q.x : (j & 3) == 1 ? q.y : (j & 3) == 2 ? q.z : q.w;
                bq[c][nt] = dequant8(word, s2[nt][j >> 2], b2[nt][j >> 2], dq);
            }
        };
        lds_a(0, 0);
        deq_b(0, 0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (j < 7) lds_a(j + 1, (j + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            if (j < 7) deq_b(j + 1, (j + 1) & 1);
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int t = 0; t < MT; t++)
                    acc[t][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[j & 1][t], bq[j & 1][nt], acc[t][nt], 0, 0, 0);
        }
        stage(buf ^ 1, xr[(I + 1) % R]);  // past the last step this stages a copy nobody reads
        __syncthreads();
    };

#pragma unroll
    for (int i = 0; i < P; i++) issue(min(s_lo + i, s_hi - 1), wlo[i], whi[i], sr[i], xr[i]);
    stage(0, xr[0]);
    __syncthreads();

    int st = s_lo;
    for (; st + R <= s_hi; st += R) {
        step(st + 0, std::integral_constant<int, 0>{});
        if constexpr (R > 1) step(st + 1, std::integral_constant<int, 1 % R>{});
        if constexpr (R > 2) step(st + 2, std::integral_constant<int, 2 % R>{});
        if constexpr (R > 3) step(st + 3, std::integral_constant<int, 3 % R>{});
        if constexpr (R > 4) step(st + 4, std::integral_constant<int, 4 % R>{});
        if constexpr (R > 5) step(st + 5, std::integral_constant<int, 5 % R>{});
    }
    // tail: fewer than R steps remain; slot of step st + i is i
    if (st < s_hi) step(st, std::integral_constant<int, 0>{});
    if constexpr (R > 2) if (st + 1 < s_hi) step(st + 1, std::integral_constant<int, 1 % R>{});
    if constexpr (R > 3) if (st + 2 < s_hi) step(st + 2, std::integral_constant<int, 2 % R>{});
    if constexpr (R > 4) if (st + 3 < s_hi) step(st + 3, std::integral_constant<int, 3 % R>{});
    if constexpr (R > 5) if (st + 4 < s_hi) step(st + 4, std::integral_constant<int, 4 % R>{});
    store_acc32<MT, NT>(a, acc, m0, col0, sp, lane);
}

// Row-major epilogue of the packed kernels (one 32-column tile per wave
// slot).  The accumulators go to LDS as row-major tiles [slot][t][32 rows]
// [kRowStride floats] (lane L, element i -> row 8*(i/4) + 4*(L/32) + i%4,
// column L%32); a row stride of 40 floats puts the two half-waves of each
// LDS access on disjoint banks.  Then every thread finishes four consecutive
// columns of a row per step (eight lanes per 128-byte row piece): split
// partials as one 16-byte store, STORE / RESIDUAL / SwiGLU with 8- or
// 16-byte accesses, instead of sixteen scattered element stores per tile.
constexpr int kRowStride = 40;

template <int MT>
__device__ __forceinline__ void acc_to_rows(const floatx16 (&acc)[MT][1], float *tile0, int lane, bool add) {
    const int hr = 4 * (lane >> 5);
    const int c = lane & 31;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float *p = tile0 + (t * 32 + 8 * (i >> 2) + hr + (i & 3)) * kRowStride + c;
            *p = add ? *p + acc[t][0][i] : acc[t][0][i];
        }
}

__device__ __forceinline__ void store4_dt(void *y, int64_t i, const float (&v)[4], int dt) {
    if (dt == VX_F32) {
        *(float4 *)((float *)y + i) = make_float4(v[0], v[1], v[2], v[3]);
        return;
    }
    uint16_t h[4];
#pragma unroll
    for (int e = 0; e < 4; e++) h[e] = dt == VX_F16 ? f32_to_f16_bits(v[e]) : f32_to_bf16_bits(v[e]);
    *(uint2 *)((uint16_t *)y + i) = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
}

__device__ __forceinline__ void load4_dt(const void *p, int64_t i, float (&v)[4], int dt) {
    if (dt == VX_F32) {
        const float4 f = *(const float4 *)((const float *)p + i);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
        return;
    }
    const uint2 w = *(const uint2 *)((const uint16_t *)p + i);
    const uint16_t h[4] = {(uint16_t)(w.x & 0xffffu), (uint16_t)(w.x >> 16), (uint16_t)(w.y & 0xffffu),
                           (uint16_t)(w.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = dt == VX_F16 ? f16_bits_to_f32(h[e]) : bf16_bits_to_f32(h[e]);
}

// Finish the row-major tiles of one workgroup (THREADS threads): columns
// colb + 32*slot + 4*c4 .. +3 of rows m0 + 32t + r.
template <int MT, int THREADS>
__device__ __forceinline__ void finish_rows(const QmmArgs &a, const float *lds, int m0, int colb, int sp, int tid,
                                            bool live) {
    if (!live) return;
    const bool partial = a.splits > 1 || a.epi == kEpiPartial;
    if (a.epi == VX_EPI_SWIGLU && !partial) {
        // per (slot, t, r): features 16*tile + 4*c4 .. +3, gate at columns
        // 4*c4 .. and up at 16 + 4*c4 .. of the tile
        constexpr int PIECES = 4 * MT * 32 * 4;
#pragma unroll
        for (int k = 0; k < (PIECES + THREADS - 1) / THREADS; k++) {
            const int e = tid + THREADS * k;
            if (PIECES % THREADS != 0 && e >= PIECES) break;
            const int slot = e / (128 * MT);
            const int t = (e >> 7) % MT;
            const int r = (e >> 2) & 31;
            const int c4 = e & 3;
            const int row = m0 + 32 * t + r;
            const int tile = colb / 32 + slot;
            if (row >= a.M || tile * 32 >= a.N) continue;
            const float *src = lds + ((slot * MT + t) * 32 + r) * kRowStride + 4 * c4;
            const float4 g4 = *(const float4 *)src, u4 = *(const float4 *)(src + 16);
            const float gv[4] = {g4.x, g4.y, g4.z, g4.w}, uv[4] = {u4.x, u4.y, u4.z, u4.w};
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float g = round_dt(gv[q] * a.acc_scale, a.round_dt);
                const float u = round_dt(uv[q] * a.acc_scale, a.round_dt);
                v[q] = round_dt(round_dt(silu_f(g), a.round_dt) * u, a.round_dt) * a.store_scale;
            }
            store4_dt(a.y, (int64_t)row * (a.N / 2) + tile * 16 + 4 * c4, v, a.y_dt);
        }
        return;
    }
    constexpr int PIECES = 4 * MT * 32 * 8;
    const bool amax = a.amax_v != nullptr && !partial;
#pragma unroll
    for (int k = 0; k < (PIECES + THREADS - 1) / THREADS; k++) {
        const int e = tid + THREADS * k;
        if (PIECES % THREADS != 0 && e >= PIECES) break;
        const int slot = e / (256 * MT);
        const int t = (e >> 8) % MT;
        const int r = (e >> 3) & 31;
        const int c4 = e & 7;
        const int row = m0 + 32 * t + r;
        const int col = colb + slot * 32 + 4 * c4;
        const bool ok = row < a.M && col < a.N;
        const float4 s4 = *(const float4 *)(lds + ((slot * MT + t) * 32 + r) * kRowStride + 4 * c4);
        if (partial) {
            if (ok) *(float4 *)(a.partial + ((int64_t)sp * a.M + row) * a.N + col) = s4;
            continue;
        }
        const int64_t idx = (int64_t)row * a.N + col;
        const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
        float v[4], rv[4];
        if (ok && a.epi == VX_EPI_RESIDUAL) load4_dt(a.resid, idx, rv, a.y_dt);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v[q] = round_dt(sv[q] * a.acc_scale, a.round_dt);
            if (a.epi == VX_EPI_RESIDUAL) v[q] = round_dt(rv[q] + v[q], a.round_dt);
            v[q] *= a.store_scale;
        }
        if (ok) store4_dt(a.y, idx, v, a.y_dt);
        if (amax) {
            // argmax over the stored values of the 32-column tile: the eight
            // lanes of a row piece are lanes e % 8 of one wave (THREADS and
            // the piece stride are multiples of 64); the tile winners meet in
            // LDS past the row-major tiles
            float bv = -__builtin_inff();
            uint32_t bi = 0xffffffffu;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float x = round_dt(v[q], a.y_dt);
                if (ok && x > bv) {  // strict: the first index wins ties; NaN never wins
                    bv = x;
                    bi = (uint32_t)(col + q);
                }
            }
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) {
                const float ov = __shfl_xor(bv, o);
                const uint32_t oi = (uint32_t)__shfl_xor((int)bi, o);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            if (c4 == 0) {
                float *wv = (float *)lds + 4 * MT * 32 * kRowStride;
                uint32_t *wi = (uint32_t *)(wv + 4 * MT * 32);
                wv[slot * MT * 32 + t * 32 + r] = bv;
                wi[slot * MT * 32 + t * 32 + r] = bi;
            }
        }
    }
    if (amax) {
        // one (value, first index) per row and workgroup (128 columns), at
        // [row * ceil(N/128) + column block]; slots combine in column order
        __syncthreads();
        const float *wv = lds + 4 * MT * 32 * kRowStride;
        const uint32_t *wi = (const uint32_t *)(wv + 4 * MT * 32);
        for (int rl = tid; rl < MT * 32; rl += THREADS) {
            const int row = m0 + rl;
            if (row >= a.M) continue;
            float bv = -__builtin_inff();
            uint32_t bi = 0xffffffffu;
#pragma unroll
            for (int slot = 0; slot < 4; slot++) {
                if (colb + slot * 32 >= a.N) break;
                const float ov = wv[slot * MT * 32 + rl];
                const uint32_t oi = wi[slot * MT * 32 + rl];
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            const int64_t at = (int64_t)row * ((a.N + 127) / 128) + colb / 128;
            a.amax_v[at] = bv;
            a.amax_i[at] = bi;
        }
    }
}

typedef __attribute__((address_space(3))) void lds_void_t;

// 16-byte LDS read at a byte address, issued outside the compiler's model of
// LDS.  Activations reach LDS by DMA (global_load_lds), and the compiler
// guards every LDS read it can see with a full vmcnt(0) after such a DMA,
// which would drain the whole prefetch ring each step.  The caller orders the
// read after its own vmcnt wait and barrier, and waits with lgkm_wait before
// using the result.
template <int OFF>
__device__ __forceinline__ half8_t lds_read16(uint32_t addr) {
    uint4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return __builtin_bit_cast(half8_t, v);
}

// s_waitcnt lgkmcnt(N), then an empty asm over the fragments so that their
// uses cannot be scheduled above the wait.
template <int N, int MT>
__device__ __forceinline__ void lgkm_wait(half8_t (&f)[MT]) {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N));
#pragma unroll
    for (int t = 0; t < MT; t++) asm volatile("" : "+v"(f[t]));
}

// One lane-strided DMA of 16 bytes per lane from global memory into LDS
// (lane l lands at lds + 16 l), also outside the compiler's view: were the
// compiler to see an LDS DMA among its pending loads, it would answer every
// later wait with vmcnt(0).  vm_wait orders it.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "m0");
}

// vm_wait<steps * (live + UW)> for a wave-uniform live count 0..UX (UX <= 3)
template <int STEPS, int UX, int UW>
__device__ __forceinline__ void vm_wait_live(int live) {
    static_assert(UX <= 3, "up to three DMA instructions per wave and step");
    if (live >= UX) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"(STEPS * (UX + UW)));
    } else if (UX >= 2 && live == UX - 1) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"(STEPS * (UX - 1 + UW)));
    } else if (UX >= 3 && live == UX - 2) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"(STEPS * (UX - 2 + UW)));
    } else {
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"(STEPS * UW));
    }
}

template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N));
}

// The packed GEMM with the activations staged by LDS DMA.  Same tiles and
// weight stream as qmm_f16_p32_kernel; the difference is where step s+P's
// activations wait: in one of P+1 LDS buffers (global_load_lds_dwordx4, no
// registers), so the prefetch depth no longer costs VGPRs and no VGPR->LDS
// copy is issued.  Per step and wave: 2*MT DMA instructions, each filling
// 1 KB = four 256-byte activation rows (row r, chunk c at r*16 + (c ^ r%16),
// the bank-spread layout), then 3*NT weight loads into the register ring.
// Step s begins with vmcnt((P-1) * (2*MT + 3*NT)): step s's DMA and weights
// have landed while the P-1 later steps stay in flight; a barrier then makes
// every wave's DMA visible and proves that the buffer refilled next was
// read to the end by everyone.
template <int MT, int NT, int P>
// leading scalars: the prologue's arguments, preloaded into SGPRs (see
// qmm_f16_k2_kernel)
__global__ __launch_bounds__(256) void qmm_f16_dma_kernel(const uint16_t *x_arg, const uint8_t *w_arg, int M_arg,
                                                          int N_arg, int K_arg, int S_arg, int sps_arg,
                                                          int splits_arg, int per_xcd_arg, int total_items_arg,
                                                          QmmArgs a) {
    constexpr int R = P + 1;
    static_assert(R >= 2 && R <= 6, "ring of 2..6 slots");
    constexpr int UX = 2 * MT;             // DMA instructions per wave per step
    constexpr int UW = 3 * NT;             // weight loads per wave per step
    constexpr int BUF = MT * 512;          // 16-byte slots per buffer (MT * 32 rows x 16 chunks)
    constexpr int VM = (P - 1) * (UX + UW);
    static_assert(VM < 64, "vmcnt range");
    __shared__ __align__(256) uint4 xs[R * BUF];

    const int bid = blockIdx.x;
    const int item = (bid & 7) * per_xcd_arg + (bid >> 3);
    if (item >= total_items_arg) return;
    const int cb = item / splits_arg;
    const int sp = item - cb * splits_arg;
    const int m0 = blockIdx.y * MT * 32;
    const int s_lo = sp * sps_arg;
    const int s_hi = min(S_arg, s_lo + sps_arg);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col0 = cb * (kWaves * NT * 32) + wave * NT * 32 + (lane & 31);

    // DMA instruction g of wave w fills slots [64 (4g + w), +64): lane l takes
    // row 16g + 4w + l/16 and chunk (l%16) ^ (row%16).  Rows past M re-read
    // row M-1 (finite values whose results are never stored).
    const uint16_t *xh = x_arg;
    int xoff[UX];
    {
        const int rl = 4 * wave + (lane >> 4);
        const int c = (lane & 15) ^ (rl & 15);
#pragma unroll
        for (int g = 0; g < UX; g++) xoff[g] = min(m0 + 16 * g + rl, M_arg - 1) * K_arg + 8 * c;
    }
    // fragment (j, t) of lane L: row 32t + L%32, chunk 2j + L/32, at byte
    // 8192 t + 256 (L%32) + 16 ((2j + L/32) ^ L%16) = 8192 t + (xrd ^ 32j)
    const uint32_t xs_addr = (uint32_t)(uintptr_t)(lds_void_t *)xs;
    const uint32_t xs_wave = __builtin_amdgcn_readfirstlane(xs_addr + wave * 64 * 16);
    const uint32_t xrd = xs_addr + (lane & 31) * 256 + 16 * ((lane >> 5) ^ (lane & 15));

    const uint8_t *wblk[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int tile = min(col0 / 32 + nt, N_arg / 32 - 1);
        wblk[nt] = w_arg + (int64_t)tile * S_arg * kPackBlock;
    }
    constexpr uint32_t kLoHalf = 0x01000100u, kHiHalf = 0x03020302u;
    const DqConst dq = dq_const();

    floatx16 acc[MT][NT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[t][nt][i] = 0.f;

    uint4 wlo[R][NT], whi[R][NT];
    uint2 sr[R][NT];

    auto issue = [&](int st, int buf, uint4 (&w0)[NT], uint4 (&w1)[NT], uint2 (&sv)[NT]) {
#pragma unroll
        for (int g = 0; g < UX; g++)
            dma16(xh + xoff[g] + st * 128, xs_wave + (uint32_t)(buf * BUF + 256 * g) * 16);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const uint8_t *bp = wblk[nt] + (int64_t)st * kPackBlock;
            w0[nt] = *(const uint4 *)(bp + lane * 16);
            w1[nt] = *(const uint4 *)(bp + 1024 + lane * 16);
            sv[nt] = *(const uint2 *)(bp + 2048 + (lane & 31) * 8);
        }
    };
    auto step = [&](int st, auto slot_c) {
        constexpr int I = decltype(slot_c)::value;
        constexpr int NX = (I + P) % R;
        vm_wait<VM>();
        __builtin_amdgcn_s_barrier();
        issue(min(st + P, s_hi - 1), NX, wlo[NX], whi[NX], sr[NX]);
        __builtin_amdgcn_sched_barrier(0);
        half2_t s2[NT][2], b2[NT][2];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            s2[nt][0] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sr[I][nt].x, sr[I][nt].x, kLoHalf));
            b2[nt][0] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sr[I][nt].x, sr[I][nt].x, kHiHalf));
            s2[nt][1] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sr[I][nt].y, sr[I][nt].y, kLoHalf));
            b2[nt][1] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sr[I][nt].y, sr[I][nt].y, kHiHalf));
        }
        const uint32_t base = xrd + I * MT * 8192;
        half8_t af[2][MT], bq[2][NT];
        auto lds_a = [&](int j, int c) {
            const uint32_t ad = base ^ (32u * j);
            if constexpr (MT > 0) af[c][0] = lds_read16<0>(ad);
            if constexpr (MT > 1) af[c][1] = lds_read16<8192>(ad);
            if constexpr (MT > 2) af[c][2] = lds_read16<16384>(ad);
        };
        auto deq_b = [&](int j, int c) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const uint4 q = (j >> 2) ? whi[I][nt] : wlo[I][nt];
                const uint32_t word = (j & 3) == 0 ? q.x : (j & 3) == 1 ? q.y : (j & 3) == 2 ? q.z : q.w;
                bq[c][nt] = dequant8(word, s2[nt][j >> 2], b2[nt][j >> 2], dq);
            }
        };
        lds_a(0, 0);
        deq_b(0, 0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            // sub-step j+1's fragments are requested before sub-step j's MFMAs,
            // whose own fragments are then waited for (MT reads stay in flight)
            if (j < 7) {
                lds_a(j + 1, (j + 1) & 1);
                lgkm_wait<MT, MT>(af[j & 1]);
            } else {
                lgkm_wait<0, MT>(af[j & 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (j < 7) deq_b(j + 1, (j + 1) & 1);
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int t = 0; t < MT; t++)
                    acc[t][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[j & 1][t], bq[j & 1][nt], acc[t][nt], 0, 0, 0);
        }
    };

#pragma unroll
    for (int i = 0; i < P; i++) issue(min(s_lo + i, s_hi - 1), i, wlo[i], whi[i], sr[i]);

    int st = s_lo;
    for (; st + R <= s_hi; st += R) {
        step(st + 0, std::integral_constant<int, 0>{});
        if constexpr (R > 1) step(st + 1, std::integral_constant<int, 1 % R>{});
        if constexpr (R > 2) step(st + 2, std::integral_constant<int, 2 % R>{});
        if constexpr (R > 3) step(st + 3, std::integral_constant<int, 3 % R>{});
        if constexpr (R > 4) step(st + 4, std::integral_constant<int, 4 % R>{});
        if constexpr (R > 5) step(st + 5, std::integral_constant<int, 5 % R>{});
    }
    // tail: fewer than R steps remain; slot of step st + i is i
    if (st < s_hi) step(st, std::integral_constant<int, 0>{});
    if constexpr (R > 2) if (st + 1 < s_hi) step(st + 1, std::integral_constant<int, 1 % R>{});
    if constexpr (R > 3) if (st + 2 < s_hi) step(st + 2, std::integral_constant<int, 2 % R>{});
    if constexpr (R > 4) if (st + 3 < s_hi) step(st + 3, std::integral_constant<int, 3 % R>{});
    if constexpr (R > 5) if (st + 4 < s_hi) step(st + 4, std::integral_constant<int, 4 % R>{});
    // the clamped prefetches past the last step still write LDS: drain them
    // before the workgroup's LDS can be handed to another workgroup
    vm_wait<0>();
    if constexpr (NT == 1 && R * BUF * 16 >= 4 * MT * 32 * kRowStride * 4 + 4 * MT * 32 * 8) {
        __syncthreads();
        acc_to_rows<MT>(acc, (float *)xs + wave * MT * 32 * kRowStride, lane, false);
        __syncthreads();
        finish_rows<MT, 256>(a, (const float *)xs, m0, cb * (kWaves * 32), sp, tid, true);
    } else {
        store_acc32<MT, NT>(a, acc, m0, col0, sp, lane);
    }
}

// Rounding and stores of the eight-wave epilogue on gfx950's converts:
// v_cvt_pk_bf16_f32 and v_cvt_f16_f32 round to nearest even like the
// software rounding (a NaN stays a NaN, its payload is not kept).
template <int DT>
__device__ __forceinline__ float round_hw(float v) {
    if constexpr (DT == VX_BF16) return (float)(__bf16)v;
    else if constexpr (DT == VX_F16) return (float)(vx_half)v;
    else return v;
}
__device__ __forceinline__ void store4_hw(void *y, int64_t i, const float (&v)[4], int dt) {
    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
    typedef vx_half halfx4_t __attribute__((ext_vector_type(4)));
    if (dt == VX_F32) {
        *(float4 *)((float *)y + i) = make_float4(v[0], v[1], v[2], v[3]);
    } else if (dt == VX_BF16) {
        const bf16x4_t h = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
        *(uint2 *)((uint16_t *)y + i) = __builtin_bit_cast(uint2, h);
    } else {
        const halfx4_t h = {(vx_half)v[0], (vx_half)v[1], (vx_half)v[2], (vx_half)v[3]};
        *(uint2 *)((uint16_t *)y + i) = __builtin_bit_cast(uint2, h);
    }
}
// SiLU with the hardware reciprocal (1 ulp) in place of an IEEE division
__device__ __forceinline__ float silu_hw(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// Epilogue of the eight-wave kernel with one 32-column tile per wave pair.
// The MFMA ran with the weights as its A operand, so accumulator element i
// of lane L is row m0 + 32t + L%32, tile column 8(i/4) + 4(L/32) + i%4: each
// register quad holds four consecutive columns of one row.  The k-halves
// split the quads: half kh keeps quads kh and kh + 2 (for SwiGLU the gate
// and the up columns of the same four features) and takes the partner's sum
// of them from LDS (own + partner, the same sum either way round).  Each
// wave then finishes its quads from registers: 16-byte f32 partials, 8-byte
// f16 / bf16 outputs, no row-major staging.  RDT is the rounding dtype.
template <int RDT, int MT>
__device__ __forceinline__ void k2_finish(const QmmArgs &a, const floatx16 (&acc)[MT][1], float4 *xs, int m0,
                                          int colb, int sp, int kh, int wc, int lane, int tid, bool live) {
    const int h = lane >> 5;
    const int tile = colb / 32 + wc;
    const bool tile_ok = live && tile * 32 < a.N;
    // hand over the quads the partner keeps: (1 - kh) + 2j
    float4 *mine = xs + (wc * 2 + kh) * MT * 2 * 64 + lane;
    const float4 *theirs = xs + (wc * 2 + (kh ^ 1)) * MT * 2 * 64 + lane;
    __syncthreads();  // every wave is past its last read of the activation ring
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int g0 = 4 * (2 * j), g1 = 4 * (1 + 2 * j);
            mine[(t * 2 + j) * 64] = kh ? make_float4(acc[t][0][g0], acc[t][0][g0 + 1], acc[t][0][g0 + 2], acc[t][0][g0 + 3])
                                        : make_float4(acc[t][0][g1], acc[t][0][g1 + 1], acc[t][0][g1 + 2], acc[t][0][g1 + 3]);
        }
    __syncthreads();
    // own quads kh + 2j, summed with the partner's
    float v[MT][2][4];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int g0 = 4 * (2 * j), g1 = 4 * (1 + 2 * j);
            const float4 o = theirs[(t * 2 + j) * 64];
            const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
            for (int q = 0; q < 4; q++) v[t][j][q] = (kh ? acc[t][0][g1 + q] : acc[t][0][g0 + q]) + ov[q];
        }
    const bool partial = a.splits > 1 || a.epi == kEpiPartial;
    if (a.epi == VX_EPI_SWIGLU && !partial) {
        // features 16 tile + 8 kh + 4h + q: gate in quad kh, up in quad kh + 2
        const int f0 = 16 * tile + 8 * kh + 4 * h;
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int row = m0 + 32 * t + (lane & 31);
            if (!tile_ok || row >= a.M) continue;
            float o[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float g = round_hw<RDT>(v[t][0][q] * a.acc_scale);
                const float u = round_hw<RDT>(v[t][1][q] * a.acc_scale);
                o[q] = round_hw<RDT>(round_hw<RDT>(silu_hw(g)) * u) * a.store_scale;
            }
            store4_hw(a.y, (int64_t)row * (a.N / 2) + f0, o, a.y_dt);
        }
        return;
    }
    const bool amax = a.amax_v != nullptr && !partial;
    float *cand_v = (float *)(xs + 4 * 2 * MT * 2 * 64);
    uint32_t *cand_i = (uint32_t *)(cand_v + 8 * MT * 32);
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int row = m0 + 32 * t + (lane & 31);
        const bool ok = tile_ok && row < a.M;
        float bv = -__builtin_inff();
        uint32_t bi = 0xffffffffu;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = tile * 32 + 8 * (kh + 2 * j) + 4 * h;
            if (partial) {
                if (ok) *(float4 *)(a.partial + ((int64_t)sp * a.M + row) * a.N + col) =
                    make_float4(v[t][j][0], v[t][j][1], v[t][j][2], v[t][j][3]);
                continue;
            }
            const int64_t idx = (int64_t)row * a.N + col;
            float rv[4] = {0.f, 0.f, 0.f, 0.f}, o[4];
            if (ok && a.epi == VX_EPI_RESIDUAL) load4_dt(a.resid, idx, rv, a.y_dt);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float x = round_hw<RDT>(v[t][j][q] * a.acc_scale);
                if (a.epi == VX_EPI_RESIDUAL) x = round_hw<RDT>(rv[q] + x);
                o[q] = x * a.store_scale;
            }
            if (ok) store4_hw(a.y, idx, o, a.y_dt);
            if (amax) {
                // columns ascend with j and q: strict > keeps the first index
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float x = round_dt(o[q], a.y_dt);
                    if (ok && x > bv) {  // NaN never wins
                        bv = x;
                        bi = (uint32_t)(col + q);
                    }
                }
            }
        }
        if (amax) {
            // the other half-wave holds the same row's other columns
            const float ov = __shfl_xor(bv, 32);
            const uint32_t oi = (uint32_t)__shfl_xor((int)bi, 32);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
            if (h == 0) {
                cand_v[((wc * 2 + kh) * MT + t) * 32 + lane] = bv;
                cand_i[((wc * 2 + kh) * MT + t) * 32 + lane] = bi;
            }
        }
    }
    if (amax) {
        // one (value, first index) per row and workgroup (128 columns) at
        // [row * ceil(N/128) + column block]: the best of the eight waves'
        // candidates (the order-free rule: larger value, then smaller index)
        __syncthreads();
        if (tid < MT * 32 && live) {
            const int row = m0 + tid;
            if (row < a.M) {
                float bv = -__builtin_inff();
                uint32_t bi = 0xffffffffu;
#pragma unroll
                for (int w = 0; w < 8; w++) {
                    const float ov = cand_v[(w * MT + tid / 32) * 32 + tid % 32];
                    const uint32_t oi = cand_i[(w * MT + tid / 32) * 32 + tid % 32];
                    if (ov > bv || (ov == bv && oi < bi)) {
                        bv = ov;
                        bi = oi;
                    }
                }
                const int64_t at = (int64_t)row * ((a.N + 127) / 128) + colb / 128;
                a.amax_v[at] = bv;
                a.amax_i[at] = bi;
            }
        }
    }
}

// The packed GEMM on eight waves: waves w and w+4 share the 32-column tiles
// of slot w%4 and split each 128-wide k step, the first taking MFMAs 0..3
// (packed words 0..3, the step's first scale group), the second MFMAs 4..7.
// Two waves per SIMD then hide each other's LDS and dequant latency, a step
// costs half the MFMA chain of the four-wave kernel, and each wave streams
// half the weight bytes.  Activations arrive by LDS DMA as in
// qmm_f16_dma_kernel (MT DMA instructions per wave per step); the two
// halves' accumulators meet in LDS once, at the end.  No early exit:
// surplus workgroups of the last XCD row recompute the last item and store
// nothing, so every kernel argument is requested in one batch at entry.
template <int MT, int NT, int P>
// The arguments the prologue needs before its first DMA come first, as
// scalars: the compiler marks them for preloading into SGPRs at wave launch
// (gfx950 kernarg preload), so the first requests do not wait on a load of
// the argument block; the epilogue's fields arrive in `a` meanwhile.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void qmm_f16_k2_kernel(
    const uint16_t *x_arg, const uint8_t *w_arg, int M_arg, int N_arg, int K_arg, int S_arg, int sps_arg,
    int splits_arg, int per_xcd_arg, int total_items_arg, QmmArgs a) {
    constexpr int R = P + 1;
    static_assert(R >= 2 && R <= 6, "ring of 2..6 slots");
    constexpr int UX = MT;
    constexpr int UW = 2 * NT;
    constexpr int BUF = MT * 512;
    constexpr int VM = (P - 1) * (UX + UW);
    static_assert(VM < 64, "vmcnt range");
    constexpr int XSLOTS = R * BUF;
    constexpr int CSLOTS = 4 * MT * NT * 16 * 64 / 4;  // float4 slots of the pair combine
    constexpr int RSLOTS = 8 * MT * 2 * 64 + 8 * MT * 32 * 2 / 4;  // ... of k2_finish: quads + argmax candidates
    constexpr int ESLOTS = CSLOTS > RSLOTS ? CSLOTS : RSLOTS;
    __shared__ __align__(256) uint4 xs[XSLOTS > ESLOTS ? XSLOTS : ESLOTS];

    const int bid = blockIdx.x;
    const int item0 = (bid & 7) * per_xcd_arg + (bid >> 3);
    const bool live = item0 < total_items_arg;
    const int item = live ? item0 : total_items_arg - 1;
    const int cb = item / splits_arg;
    const int sp = item - cb * splits_arg;
    const int m0 = blockIdx.y * MT * 32;
    const int s_lo = sp * sps_arg;
    const int s_hi = min(S_arg, s_lo + sps_arg);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = wave >> 2;
    const int wc = wave & 3;
    const int col0 = cb * (kWaves * NT * 32) + wc * NT * 32 + (lane & 31);

    // DMA instruction g of wave w fills slots [64 (8g + w), +64): lane l takes
    // row 32g + 4w + l/16, chunk (l%16) ^ (row%16).  Rows past M re-read row M-1.
    const uint16_t *xh = x_arg;
    int xoff[UX];
    {
        const int rl = 4 * wave + (lane >> 4);
        const int c = (lane & 15) ^ (rl & 15);
#pragma unroll
        for (int g = 0; g < UX; g++) xoff[g] = min(m0 + 32 * g + rl, M_arg - 1) * K_arg + 8 * c;
    }
    // DMA instructions whose four rows all lie past M are skipped (those LDS
    // rows only feed accumulator rows that are never stored); the count of
    // live ones is wave-uniform and selects the step's vmcnt immediate
    const int nx = min(UX, max(0, (M_arg - m0 - 4 * wave + 31) / 32));
    const uint32_t xs_addr = (uint32_t)(uintptr_t)(lds_void_t *)xs;
    const uint32_t xs_wave = __builtin_amdgcn_readfirstlane(xs_addr + wave * 64 * 16);
    // fragment (j, t), j = 4 kh + jj: byte 8192 t + (xrd ^ 32 j)
    const uint32_t xrd = (xs_addr + (lane & 31) * 256 + 16 * ((lane >> 5) ^ (lane & 15))) ^ (128u * kh);

    const uint8_t *wblk[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int tile = min(col0 / 32 + nt, N_arg / 32 - 1);
        wblk[nt] = w_arg + (int64_t)tile * S_arg * kPackBlock;
    }
    const int wq_off = kh * 1024 + lane * 16;
    const int sb_off = 2048 + (lane & 31) * 8 + kh * 4;
    constexpr uint32_t kLoHalf = 0x01000100u, kHiHalf = 0x03020302u;
    const DqConst dq = dq_const();

    floatx16 acc[MT][NT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[t][nt][i] = 0.f;

    uint4 wq[R][NT];
    uint32_t sb[R][NT];

    auto issue = [&](int st, int buf, uint4 (&w)[NT], uint32_t (&sv)[NT]) {
#pragma unroll
        for (int g = 0; g < UX; g++)
            if (g < nx) dma16(xh + xoff[g] + st * 128, xs_wave + (uint32_t)(buf * BUF + 512 * g) * 16);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const uint8_t *bp = wblk[nt] + (int64_t)st * kPackBlock;
            w[nt] = *(const uint4 *)(bp + wq_off);
            sv[nt] = *(const uint32_t *)(bp + sb_off);
        }
    };
    auto step = [&](int st, auto slot_c) {
        constexpr int I = decltype(slot_c)::value;
        constexpr int NX = (I + P) % R;
        vm_wait_live<P - 1, UX, UW>(nx);
        __builtin_amdgcn_s_barrier();
        issue(min(st + P, s_hi - 1), NX, wq[NX], sb[NX]);
        __builtin_amdgcn_sched_barrier(0);
        half2_t s2[NT], b2[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            s2[nt] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sb[I][nt], sb[I][nt], kLoHalf));
            b2[nt] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(sb[I][nt], sb[I][nt], kHiHalf));
        }
        const uint32_t base = xrd + I * MT * 8192;
        half8_t af[2][MT], bq[2][NT];
        auto lds_a = [&](int jj, int c) {
            const uint32_t ad = base ^ (32u * jj);
            if constexpr (MT > 0) af[c][0] = lds_read16<0>(ad);
            if constexpr (MT > 1) af[c][1] = lds_read16<8192>(ad);
            if constexpr (MT > 2) af[c][2] = lds_read16<16384>(ad);
        };
        auto deq_b = [&](int jj, int c) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const uint4 q = wq[I][nt];
                const uint32_t word = jj == 0 ? q.x : jj == 1 ? q.y : jj == 2 ? q.z : q.w;
                bq[c][nt] = dequant8(word, s2[nt], b2[nt], dq);
            }
        };
        lds_a(0, 0);
        deq_b(0, 0);
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            if (jj < 3) {
                lds_a(jj + 1, (jj + 1) & 1);
                lgkm_wait<MT, MT>(af[jj & 1]);
            } else {
                lgkm_wait<0, MT>(af[jj & 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (jj < 3) deq_b(jj + 1, (jj + 1) & 1);
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    // one column tile per wave: weights as the A operand, so
                    // each register quad holds four columns of one row
                    if constexpr (NT == 1)
                        acc[t][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bq[jj & 1][nt], af[jj & 1][t], acc[t][nt], 0, 0, 0);
                    else
                        acc[t][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[jj & 1][t], bq[jj & 1][nt], acc[t][nt], 0, 0, 0);
                }
        }
    };

#pragma unroll
    for (int i = 0; i < P; i++) issue(min(s_lo + i, s_hi - 1), i, wq[i], sb[i]);

    int st = s_lo;
    for (; st + R <= s_hi; st += R) {
        step(st + 0, std::integral_constant<int, 0>{});
        if constexpr (R > 1) step(st + 1, std::integral_constant<int, 1 % R>{});
        if constexpr (R > 2) step(st + 2, std::integral_constant<int, 2 % R>{});
        if constexpr (R > 3) step(st + 3, std::integral_constant<int, 3 % R>{});
        if constexpr (R > 4) step(st + 4, std::integral_constant<int, 4 % R>{});
        if constexpr (R > 5) step(st + 5, std::integral_constant<int, 5 % R>{});
    }
    if (st < s_hi) step(st, std::integral_constant<int, 0>{});
    if constexpr (R > 2) if (st + 1 < s_hi) step(st + 1, std::integral_constant<int, 1 % R>{});
    if constexpr (R > 3) if (st + 2 < s_hi) step(st + 2, std::integral_constant<int, 2 % R>{});
    if constexpr (R > 4) if (st + 3 < s_hi) step(st + 3, std::integral_constant<int, 3 % R>{});
    if constexpr (R > 5) if (st + 4 < s_hi) step(st + 4, std::integral_constant<int, 4 % R>{});
    vm_wait<0>();

    if constexpr (NT == 1) {
        float4 *ex = (float4 *)xs;
        if (a.round_dt == VX_BF16)
            k2_finish<VX_BF16, MT>(a, acc, ex, m0, cb * (kWaves * 32), sp, kh, wc, lane, tid, live);
        else if (a.round_dt == VX_F16)
            k2_finish<VX_F16, MT>(a, acc, ex, m0, cb * (kWaves * 32), sp, kh, wc, lane, tid, live);
        else
            k2_finish<VX_F32, MT>(a, acc, ex, m0, cb * (kWaves * 32), sp, kh, wc, lane, tid, live);
        return;
    }

    // pair combine: the k-half-1 wave of slot wc hands its accumulators to the
    // k-half-0 wave through LDS (float4 slot ((wc, t, nt) * 4 + q) * 64 + lane)
    __syncthreads();
    float4 *cs = (float4 *)xs;
    if (kh == 1) {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    cs[(((wc * MT + t) * NT + nt) * 4 + q) * 64 + lane] =
                        make_float4(acc[t][nt][4 * q], acc[t][nt][4 * q + 1], acc[t][nt][4 * q + 2], acc[t][nt][4 * q + 3]);
    }
    __syncthreads();
    if (kh == 0 && live) {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 o = cs[(((wc * MT + t) * NT + nt) * 4 + q) * 64 + lane];
                    acc[t][nt][4 * q] += o.x;
                    acc[t][nt][4 * q + 1] += o.y;
                    acc[t][nt][4 * q + 2] += o.z;
                    acc[t][nt][4 * q + 3] += o.w;
                }
        store_acc32<MT, NT>(a, acc, m0, col0, sp, lane);
    }
}

// Split-K finish: sum the partials of each output in split order, then the
// epilogue.  One thread per output element (per (row, feature) for SwiGLU).
__global__ __launch_bounds__(256) void qmm_reduce_kernel(QmmArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (a.epi == VX_EPI_SWIGLU) {
        const int64_t half = a.N / 2;
        if (idx >= (int64_t)a.M * half) return;
        const int row = (int)(idx / half);
        const int f = (int)(idx - (int64_t)row * half);
        const int gcol = (f / 16) * 32 + (f % 16);
        float g = 0.f, u = 0.f;
        for (int q = 0; q < a.splits; q++) {
            const float *p = a.partial + ((int64_t)q * a.M + row) * a.N;
            g += p[gcol];
            u += p[gcol + 16];
        }
        epi_swiglu(a, row, f, g, u);
        return;
    }
    if (idx >= (int64_t)a.M * a.N) return;
    const int row = (int)(idx / a.N);
    const int col = (int)(idx - (int64_t)row * a.N);
    float sum = 0.f;
    for (int q = 0; q < a.splits; q++) sum += a.partial[((int64_t)q * a.M + row) * a.N + col];
    epi_elem(a, row, col, sum);
}

// One thread per output, the reference's arithmetic (metal_kernels.rs:418-479):
// dequantise in f32, accumulate eight products per packed word, add bias.
template <int DT>
__global__ void qmm_naive_kernel(const void *x, const uint32_t *qw, const void *sc, const void *bs,
                                 const void *bias, void *y, int64_t m, int64_t n, int64_t k,
                                 int64_t gs) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= m * n) return;
    const int64_t mi = idx / n, ni = idx - mi * n;
    const int64_t kp = k / 8, kg = k / gs, gpp = gs / 8;
    float acc = 0.f;
    for (int64_t g = 0; g < kg; g++) {
        const float s = ld_elem<DT>(sc, ni * kg + g);
        const float b = ld_elem<DT>(bs, ni * kg + g);
        for (int64_t p = 0; p < gpp; p++) {
            const uint32_t pkg = qw[ni * kp + g * gpp + p];
            const int64_t k0 = g * gs + p * 8;
            float part = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float w = __fadd_rn(__fmul_rn((float)((pkg >> (4 * e)) & 0xFu), s), b);
                part += ld_elem<DT>(x, mi * k + k0 + e) * w;
            }
            acc += part;
        }
    }
    if (bias) acc += ld_elem<DT>(bias, ni);
    st_elem<DT>(y, idx, acc);
}


struct Plan {
    bool stream;  // f16 streaming kernel (else the LDS-chunked kernel)
    bool p32;     // packed weights on the 32x32 MFMA kernel
    bool k2;      // ... on its eight-wave, k-split form
    int MT, NT, P, splits, gps, sps, col_blocks, m_blocks, per_xcd, total_items;
    size_t partial_bytes;
};

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// Prefetch depth of the streaming kernel by row-tile count: the register ring
// holds P+1 steps of weights and activations.
constexpr int stream_depth(int mt) { return mt <= 2 ? 4 : 3; }

// Prefetch depth of the packed kernel by tile counts (register budget).
constexpr int p32_depth(int mt, int nt) { return mt == 1 ? 4 : (mt == 2 ? 3 : (nt == 1 ? 2 : 1)); }

// Packed-weight plan: 32-row tiles (up to 3 per workgroup), 32-column tiles.
Plan make_plan_p32(int64_t M, int64_t N, int64_t K, int epi) {
    Plan p{};
    p.stream = true;
    p.p32 = true;
    const int cus = device_cu_count();
    p.MT = (int)std::min<int64_t>(3, std::max<int64_t>(1, vx_cdiv(std::min<int64_t>(M, 96), 32)));
    p.m_blocks = (int)vx_cdiv(M, p.MT * 32);
    const int S = (int)(K / 128);
    int nt = env_int("VX_QMM_NT", 1);
    p.NT = nt;
    p.P = p32_depth(p.MT, nt);
    // the eight-wave kernel for three row tiles (verify rows) and for one row
    // tile below LM-head widths (measured in the spec bench: the four-wave
    // kernel is faster only for the draft's one-row-tile LM head)
    const int k2_env = env_int("VX_QMM_K2", -1);
    p.k2 = k2_env >= 0 ? k2_env != 0 : (nt == 1 && (p.MT == 3 || (p.MT == 1 && N <= 65536)));
    p.col_blocks = (int)vx_cdiv(N, kWaves * nt * 32);
    const int items = p.col_blocks * p.m_blocks;
    // three row tiles hold one workgroup per CU (registers); fewer hold two.
    // Partial mode aims a little lower: its consumer reads every split.
    const double per_cu = p.k2 ? env_int("VX_QMM_PERCU", 1) : (p.MT >= 3 ? 1.0 : 2.0);
    const double target = per_cu * cus * (epi == kEpiPartial ? 0.9 : 1.0);
    int splits = std::max(1, (int)(target / std::max(1, items) + 0.5));
    if (epi == kEpiPartial) splits = std::min(splits, kMaxPartialSplits);
    // A whole-output epilogue (STORE, RESIDUAL, SwiGLU) over at least half
    // the CUs' worth of column blocks: one split on the eight-wave kernel, so
    // the epilogue runs in place and no finishing kernel is launched (gate|up
    // at M = 80 as a plain store: 20.1 us against 27.0 us with two splits and
    // the reduce kernel)
    const bool whole = epi != kEpiPartial && nt == 1 && p.MT <= env_int("VX_QMM_SWIGLU_MT", 3) && p.MT != 2 &&
                       2 * items >= cus;
    if (whole) splits = 1;
    splits = env_int("VX_QMM_SPLITS", splits);
    splits = std::max(1, std::min(splits, S));
    int sps = (int)vx_cdiv(S, splits);
    splits = (int)vx_cdiv(S, sps);
    while (splits > 1 && (size_t)splits * M * N * 4 > kMaxPartialBytes) {
        sps++;
        splits = (int)vx_cdiv(S, sps);
    }
    p.splits = splits;
    p.sps = sps;
    p.gps = 2 * sps;
    p.total_items = p.col_blocks * p.splits;
    p.per_xcd = (int)vx_cdiv(p.total_items, 8);
    p.partial_bytes = (p.splits > 1 || epi == kEpiPartial) ? (size_t)p.splits * M * N * 4 : 0;
    return p;
}

Plan make_plan(int64_t M, int64_t N, int64_t K, int epi, bool stream) {
    Plan p{};
    p.stream = stream;
    const int64_t mrows = std::min<int64_t>(M, 80);
    p.MT = (int)std::max<int64_t>(1, vx_cdiv(mrows, 16));
    p.m_blocks = (int)vx_cdiv(M, p.MT * 16);
    const int cus = device_cu_count();
    const int target = 2 * cus;
    if (stream) {
        const int S = (int)(K / 128);
        int nt = 2;
        if (epi == kEpiPartial) nt = N >= 16384 ? 2 : 1;
        while (nt > (epi == VX_EPI_SWIGLU ? 2 : 1) && vx_cdiv(N, kWaves * nt * 16) * p.m_blocks * 4 < target)
            nt /= 2;
        nt = env_int("VX_QMM_NT", nt);
        p.NT = nt;
        p.P = stream_depth(p.MT);
        p.col_blocks = (int)vx_cdiv(N, kWaves * nt * 16);
        const int items = p.col_blocks * p.m_blocks;
        // partial mode: the consumer reads every split, so aim for fewer,
        // longer workgroups (~0.7 per CU); otherwise ~2 per CU
        int splits = epi == kEpiPartial ? std::max(1, std::min(kMaxPartialSplits, (int)((0.7 * cus) / std::max(1, items) + 0.5)))
                                        : std::max(1, target / std::max(1, items));
        splits = env_int("VX_QMM_SPLITS", splits);
        splits = std::max(1, std::min(splits, S));
        int sps = (int)vx_cdiv(S, splits);
        splits = (int)vx_cdiv(S, sps);
        while (splits > 1 && (size_t)splits * M * N * 4 > kMaxPartialBytes) {
            sps++;
            splits = (int)vx_cdiv(S, sps);
        }
        p.splits = splits;
        p.sps = sps;
        p.gps = 2 * sps;
    } else {
        int nt = p.MT >= 3 ? 4 : (p.MT == 2 ? 2 : 1);
        if (epi == VX_EPI_SWIGLU) nt = std::max(nt, 2);
        const int G = (int)(K / 64);
        // prefer narrower column blocks when the grid would be too small
        while (nt > (epi == VX_EPI_SWIGLU ? 2 : 1) &&
               vx_cdiv(N, kWaves * nt * 16) * p.m_blocks * std::max(1, G / kChunkGroups) < target)
            nt /= 2;
        nt = env_int("VX_QMM_NT", nt);
        p.NT = nt;
        p.col_blocks = (int)vx_cdiv(N, kWaves * nt * 16);
        const int items = p.col_blocks * p.m_blocks;
        int splits = std::max(1, target / std::max(1, items));
        splits = std::min(splits, std::max(1, G / kChunkGroups));
        splits = env_int("VX_QMM_SPLITS", splits);
        splits = std::max(1, std::min(splits, G / kChunkGroups));
        int gps = (int)vx_cdiv(G, splits);
        gps = (int)vx_cdiv(gps, kChunkGroups) * kChunkGroups;
        splits = (int)vx_cdiv(G, gps);
        // bound the partial-sum workspace
        while (splits > 1 && (size_t)splits * M * N * 4 > kMaxPartialBytes) {
            gps += kChunkGroups;
            splits = (int)vx_cdiv(G, gps);
        }
        p.splits = splits;
        p.gps = gps;
    }
    p.total_items = p.col_blocks * p.splits;
    p.per_xcd = (int)vx_cdiv(p.total_items, 8);
    p.partial_bytes = (p.splits > 1 || epi == kEpiPartial) ? (size_t)p.splits * M * N * 4 : 0;
    return p;
}

void launch_reduce(const QmmArgs &a, const Plan &p, hipStream_t st) {
    if (p.splits > 1 && a.epi != kEpiPartial) {
        const int64_t outs = (int64_t)a.M * (a.epi == VX_EPI_SWIGLU ? a.N / 2 : a.N);
        hipLaunchKernelGGL(qmm_reduce_kernel, dim3((unsigned)vx_cdiv(outs, 256)), dim3(256), 0, st, a);
    }
}

template <int MT, int NT>
void launch_stream(const QmmArgs &a, const Plan &p, hipStream_t st) {
    dim3 grid(p.per_xcd * 8, p.m_blocks);
    hipLaunchKernelGGL((qmm_f16_stream_kernel<MT, NT, stream_depth(MT)>), grid, dim3(256), 0, st, a);
    launch_reduce(a, p, st);
}

template <int MT, int NT>
void launch_p32(const QmmArgs &a, const Plan &p, hipStream_t st) {
    dim3 grid(p.per_xcd * 8, p.m_blocks);
    hipLaunchKernelGGL((qmm_f16_p32_kernel<MT, NT, p32_depth(MT, NT)>), grid, dim3(256), 0, st, a);
    launch_reduce(a, p, st);
}

template <int MT, int NT, int P>
void launch_dma(const QmmArgs &a, const Plan &p, hipStream_t st) {
    dim3 grid(p.per_xcd * 8, p.m_blocks);
    hipLaunchKernelGGL((qmm_f16_dma_kernel<MT, NT, P>), grid, dim3(256), 0, st, (const uint16_t *)a.x,
                       (const uint8_t *)a.w, a.M, a.N, a.K, a.S, a.sps, a.splits, a.per_xcd, a.total_items, a);
    launch_reduce(a, p, st);
}

template <int MT, int NT, int P>
void launch_k2(const QmmArgs &a, const Plan &p, hipStream_t st) {
    dim3 grid(p.per_xcd * 8, p.m_blocks);
    hipLaunchKernelGGL((qmm_f16_k2_kernel<MT, NT, P>), grid, dim3(512), 0, st, (const uint16_t *)a.x,
                       (const uint8_t *)a.w, a.M, a.N, a.K, a.S, a.sps, a.splits, a.per_xcd, a.total_items, a);
    launch_reduce(a, p, st);
}

int dispatch_p32(const QmmArgs &a, const Plan &p, hipStream_t st) {
    if (p.k2) {
        const int P = env_int("VX_QMM_P", p.MT == 3 ? 2 : 3);
#define VX_KCASE(mt, nt, pp)                             \
        if (p.MT == mt && p.NT == nt && P == pp) {       \
            launch_k2<mt, nt, pp>(a, p, st);             \
            return 0;                                    \
        }
        VX_KCASE(1, 1, 2) VX_KCASE(1, 1, 3) VX_KCASE(1, 1, 4)
        VX_KCASE(2, 1, 2) VX_KCASE(2, 1, 3)
        VX_KCASE(3, 1, 2) VX_KCASE(3, 1, 3)
        VX_KCASE(1, 2, 3) VX_KCASE(3, 2, 2)
#undef VX_KCASE
        return set_error("qmm: no eight-wave kernel for tile plan");
    }
    if (env_int("VX_QMM_DMA", 1)) {
        const int P = env_int("VX_QMM_P", p.MT == 3 ? 2 : 3);
#define VX_DCASE(mt, nt, pp)                             \
        if (p.MT == mt && p.NT == nt && P == pp) {       \
            launch_dma<mt, nt, pp>(a, p, st);            \
            return 0;                                    \
        }
        VX_DCASE(1, 1, 2) VX_DCASE(1, 1, 3) VX_DCASE(1, 1, 4) VX_DCASE(1, 1, 5)
        VX_DCASE(1, 2, 2) VX_DCASE(1, 2, 3) VX_DCASE(1, 2, 4)
        VX_DCASE(2, 1, 2) VX_DCASE(2, 1, 3) VX_DCASE(2, 1, 4)
        VX_DCASE(2, 2, 2) VX_DCASE(2, 2, 3)
        VX_DCASE(3, 1, 2) VX_DCASE(3, 1, 3) VX_DCASE(3, 1, 4)
        VX_DCASE(3, 2, 2) VX_DCASE(3, 2, 3)
        VX_DCASE(3, 4, 1) VX_DCASE(3, 4, 2)
#undef VX_DCASE
        return set_error("qmm: no DMA kernel for tile plan");
    }
#define VX_CASE(mt, nt)                \
    if (p.MT == mt && p.NT == nt) {    \
        launch_p32<mt, nt>(a, p, st);  \
        return 0;                      \
    }
    VX_CASE(1, 1) VX_CASE(1, 2)
    VX_CASE(2, 1) VX_CASE(2, 2)
    VX_CASE(3, 1) VX_CASE(3, 2)
#undef VX_CASE
    return set_error("qmm: no packed kernel for tile plan");
}

int dispatch_stream(const QmmArgs &a, const Plan &p, hipStream_t st) {
#define VX_CASE(mt, nt)                   \
    if (p.MT == mt && p.NT == nt) {       \
        launch_stream<mt, nt>(a, p, st);  \
        return 0;                         \
    }
    VX_CASE(1, 1) VX_CASE(1, 2) VX_CASE(1, 4)
    VX_CASE(2, 1) VX_CASE(2, 2) VX_CASE(2, 4)
    VX_CASE(3, 1) VX_CASE(3, 2) VX_CASE(3, 4)
    VX_CASE(4, 1) VX_CASE(4, 2) VX_CASE(4, 4)
    VX_CASE(5, 1) VX_CASE(5, 2) VX_CASE(5, 4)
#undef VX_CASE
    return set_error("qmm: no streaming kernel for tile plan");
}

template <int MT, int NT, bool XBF>
void launch_fast(const QmmArgs &a, const Plan &p, hipStream_t st) {
    dim3 grid(p.per_xcd * 8, p.m_blocks);
    hipLaunchKernelGGL((qmm_int4_kernel<MT, NT, XBF>), grid, dim3(256), 0, st, a);
    launch_reduce(a, p, st);
}

template <bool XBF>
int dispatch_fast(const QmmArgs &a, const Plan &p, hipStream_t st) {
#define VX_CASE(mt, nt)                                  \
    if (p.MT == mt && p.NT == nt) {                      \
        launch_fast<mt, nt, XBF>(a, p, st);              \
        return 0;                                        \
    }
    VX_CASE(1, 1) VX_CASE(1, 2) VX_CASE(1, 4)
    VX_CASE(2, 1) VX_CASE(2, 2) VX_CASE(2, 4)
    VX_CASE(3, 1) VX_CASE(3, 2) VX_CASE(3, 4)
    VX_CASE(4, 1) VX_CASE(4, 2) VX_CASE(4, 4)
    VX_CASE(5, 1) VX_CASE(5, 2) VX_CASE(5, 4)
#undef VX_CASE
    return set_error("qmm: no kernel for tile plan");
}

// Operand requirements of the tiled kernels: f16 activations take the
// streaming kernel (K % 128, 16-byte weight rows), bf16 the LDS-chunked one.
bool fast_ok(int dt, int64_t K, int64_t gs, const void *x, const void *w, const void *s, const void *b) {
    if (gs != 64 || ((uintptr_t)x % 16) != 0) return false;
    if (dt == VX_F16)
        return K % 128 == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)s % 4) == 0 && ((uintptr_t)b % 4) == 0;
    return K % 256 == 0 && ((uintptr_t)w % 8) == 0 && ((uintptr_t)s % 8) == 0 && ((uintptr_t)b % 8) == 0;
}

}  // namespace

// Workspace of the f16 paths (row-major MLX weights, or packed weights).
size_t qmm_workspace_bytes(int64_t m, int64_t n, int64_t k, int epi, bool packed) {
    if (k % 128 != 0) return kCounterBytes;
    Plan p = packed ? make_plan_p32(m, n, k, epi) : make_plan(m, n, k, epi, true);
    return kCounterBytes + p.partial_bytes;
}

int qmm_launch(const void *x, const uint32_t *w, const void *s, const void *b, void *y,
               const void *resid, int64_t M, int64_t N, int64_t K, int x_dt, int x_shift,
               int y_shift, int round_dt, int y_dt, int epi, void *workspace, size_t ws_bytes,
               hipStream_t st, bool packed = false, float *amax_v = nullptr, uint32_t *amax_i = nullptr,
               const void *bias = nullptr) {
    Plan p = packed ? make_plan_p32(M, N, K, epi) : make_plan(M, N, K, epi, x_dt == VX_F16);
    if (epi == VX_EPI_SWIGLU && (N % 32 != 0 || (!p.p32 && p.NT % 2 != 0)))
        return set_error("qmm swiglu: N must be a multiple of 32 with paired tiles");
    void *ws = workspace;
    if (p.partial_bytes > 0) {
        if (!ws) {
            VX_TRY(stream_workspace(st, kCounterBytes + p.partial_bytes, &ws));
        } else if (ws_bytes < kCounterBytes + p.partial_bytes) {
            return set_error("qmm: workspace too small (see vx_qmm_workspace_size)");
        }
    }
    if (bias && (packed || epi != VX_EPI_STORE)) return set_error("qmm: a bias goes with the row-major STORE GEMM");
    QmmArgs a{};
    a.amax_v = amax_v;
    a.amax_i = amax_i;
    a.bias = bias;
    a.x = x;
    a.w = w;
    a.s = (const uint16_t *)s;
    a.b = (const uint16_t *)b;
    a.y = y;
    a.resid = resid;
    a.partial = ws ? (float *)((char *)ws + kCounterBytes) : nullptr;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.G = (int)(K / 64);
    a.splits = p.splits;
    a.gps = p.gps;
    a.S = (int)(K / 128);
    a.sps = p.sps;
    a.col_blocks = p.col_blocks;
    a.m_blocks = p.m_blocks;
    a.per_xcd = p.per_xcd;
    a.total_items = p.total_items;
    a.epi = epi;
    a.round_dt = round_dt;
    a.y_dt = y_dt;
    a.acc_scale = ldexpf(1.0f, x_shift);
    a.store_scale = ldexpf(1.0f, -y_shift);
    if (!p.stream && x_dt != VX_BF16) return set_error("qmm: the chunked kernel takes bf16 activations only");
    int rc = p.p32 ? dispatch_p32(a, p, st) : (p.stream ? dispatch_stream(a, p, st) : dispatch_fast<true>(a, p, st));
    if (rc) return rc;
    VX_HIP(hipGetLastError());
    return 0;
}

int qmm_fast(const void *x, const uint32_t *w, const void *s, const void *b, void *y,
             const void *resid, int64_t M, int64_t N, int64_t K, int x_dt, int x_shift,
             int round_dt, int y_dt, int epi, void *workspace, size_t ws_bytes, hipStream_t st,
             const void *bias = nullptr) {
    return qmm_launch(x, w, s, b, y, resid, M, N, K, x_dt, x_shift, 0, round_dt, y_dt, epi, workspace,
                      ws_bytes, st, false, nullptr, nullptr, bias);
}

size_t qmm_packed_bytes(int64_t n, int64_t k) { return (size_t)(n / 32) * (size_t)(k / 128) * kPackBlock; }

int qmm_pack(const uint32_t *w, const void *s, const void *b, void *out, int64_t N, int64_t K, hipStream_t st) {
    if (N % 32 != 0 || K % 128 != 0) return set_error("qmm pack: N must be a multiple of 32 and K of 128");
    if (((uintptr_t)w % 16) != 0 || ((uintptr_t)out % 16) != 0) return set_error("qmm pack: misaligned operand");
    const int64_t blocks = (N / 32) * (K / 128);
    if (blocks == 0) return 0;
    hipLaunchKernelGGL(qmm_pack_kernel, dim3((unsigned)blocks), dim3(64), 0, st, w, (const uint16_t *)s,
                       (const uint16_t *)b, (uint8_t *)out, (int)N, (int)K);
    VX_HIP(hipGetLastError());
    return 0;
}

// GEMM over packed weights (f16 activations, optionally X * 2^-x_shift; result
// scaled by 2^x_shift, rounded to round_dt, stored as value * 2^-y_shift).
int qmm_packed(const void *x, const void *packed, void *y, const void *resid, int64_t M, int64_t N, int64_t K,
               int x_shift, int y_shift, int round_dt, int y_dt, int epi, void *workspace, size_t ws_bytes,
               hipStream_t st) {
    if (N % 32 != 0 || K % 128 != 0) return set_error("qmm packed: N must be a multiple of 32 and K of 128");
    if (((uintptr_t)x % 16) != 0 || ((uintptr_t)packed % 16) != 0) return set_error("qmm packed: misaligned operand");
    return qmm_launch(x, (const uint32_t *)packed, nullptr, nullptr, y, resid, M, N, K, VX_F16, x_shift, y_shift,
                      round_dt, y_dt, epi, workspace, ws_bytes, st, true);
}

// The packed STORE GEMM with greedy-argmax partials of its stored values
// ((value, first index) per row and 128-column block, [M, N/128]): available
// when the plan runs one split on a one-tile-per-wave kernel with the
// row-major epilogue (qmm_packed_argmax_ok).
bool qmm_packed_argmax_ok(int64_t M, int64_t N, int64_t K) {
    if (N % 128 != 0 || K % 128 != 0) return false;
    const Plan p = make_plan_p32(M, N, K, VX_EPI_STORE);
    // the four-wave kernel holds the row-major tiles in its LDS ring from P = 2 on
    const bool dma_rows = env_int("VX_QMM_DMA", 1) != 0 && env_int("VX_QMM_P", p.MT == 3 ? 2 : 3) >= 2;
    return p.splits == 1 && p.NT == 1 && (p.k2 || dma_rows);
}

int qmm_packed_argmax(const void *x, const void *packed, void *y, int64_t M, int64_t N, int64_t K, int round_dt,
                      int y_dt, float *amax_v, uint32_t *amax_i, void *workspace, size_t ws_bytes, hipStream_t st) {
    if (!qmm_packed_argmax_ok(M, N, K)) return set_error("qmm packed argmax: the plan has no row-major epilogue");
    if (((uintptr_t)x % 16) != 0 || ((uintptr_t)packed % 16) != 0) return set_error("qmm packed: misaligned operand");
    return qmm_launch(x, (const uint32_t *)packed, nullptr, nullptr, y, nullptr, M, N, K, VX_F16, 0, 0, round_dt,
                      y_dt, VX_EPI_STORE, workspace, ws_bytes, st, true, amax_v, amax_i);
}

// Packed GEMM whose epilogue writes raw f32 split partials into the
// workspace (after its reserved head): partial[(sp * M + row) * N + col] for
// sp < *splits.  A fused consumer reduces them in split order.
size_t qmm_partial_ws_bytes(int64_t M, int64_t N, int64_t K) {
    if (K % 128 != 0) return kCounterBytes;
    return kCounterBytes + make_plan_p32(M, N, K, kEpiPartial).partial_bytes;
}
int qmm_packed_partial(const void *x, const void *packed, int64_t M, int64_t N, int64_t K, void *workspace,
                       size_t ws_bytes, int *splits, const float **partial, hipStream_t st) {
    if (N % 32 != 0 || K % 128 != 0) return set_error("qmm packed: N must be a multiple of 32 and K of 128");
    if (((uintptr_t)x % 16) != 0 || ((uintptr_t)packed % 16) != 0) return set_error("qmm packed: misaligned operand");
    if (!workspace) return set_error("qmm packed partial: needs a workspace");
    const Plan p = make_plan_p32(M, N, K, kEpiPartial);
    *splits = p.splits;
    *partial = (const float *)((const char *)workspace + kCounterBytes);
    return qmm_launch(x, (const uint32_t *)packed, nullptr, nullptr, nullptr, nullptr, M, N, K, VX_F16, 0, 0,
                      VX_BF16, VX_BF16, kEpiPartial, workspace, ws_bytes, st, true);
}

}  // namespace vx

using namespace vx;

extern "C" size_t vx_qmm_packed_size(int64_t n, int64_t k) { return qmm_packed_bytes(n, k); }

extern "C" int vx_qmm_pack_4bit(const uint32_t *qweight, const void *scales, const void *biases, void *packed,
                                int64_t n, int64_t k, void *stream) {
    VX_REQUIRE(qweight && scales && biases && packed, "qmm_pack_4bit: null tensor");
    return qmm_pack(qweight, scales, biases, packed, n, k, (hipStream_t)stream);
}

extern "C" int vx_qmm_4bit_packed(const void *x, const void *packed, void *y, const void *residual, int64_t m,
                                  int64_t n, int64_t k, int x_shift, int round_dtype, int y_dtype, int epilogue,
                                  void *workspace, size_t workspace_bytes, void *stream) {
    if (m == 0 || n == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(x && packed && y, "qmm_4bit_packed: null tensor");
    VX_REQUIRE(epilogue != VX_EPI_RESIDUAL || residual, "qmm_4bit_packed: residual epilogue needs R");
    return qmm_packed(x, packed, y, residual, m, n, k, x_shift, 0, round_dtype, y_dtype, epilogue, workspace,
                      workspace_bytes, (hipStream_t)stream);
}

extern "C" int vx_qmm_4bit(const void *x, const uint32_t *qweight, const void *scales,
                           const void *biases, const void *bias, void *y, int64_t m, int64_t n,
                           int64_t k, int64_t group_size, int dtype, void *stream) {
    // validation mirrors metal_kernels.rs:2082-2130
    VX_REQUIRE(k % 8 == 0, "qmm_4bit: K must be a multiple of 8");
    VX_REQUIRE(group_size != 0 && group_size % 8 == 0 && k % group_size == 0,
               "qmm_4bit: group_size must be a multiple of 8 and divide K");
    VX_REQUIRE(dtype == VX_F32 || dtype == VX_F16 || dtype == VX_BF16, "qmm_4bit: unsupported dtype");
    VX_REQUIRE(m >= 0 && n >= 0, "qmm_4bit: negative shape");
    if (m == 0 || n == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(x && qweight && scales && biases && y, "qmm_4bit: null tensor");
    hipStream_t st = (hipStream_t)stream;
    if (dtype != VX_F32 && fast_ok(dtype, k, group_size, x, qweight, scales, biases) && m * n < ((int64_t)1 << 31)) {
        // the bias joins the f32 accumulator before the one rounding to T
        return qmm_fast(x, qweight, scales, biases, y, nullptr, m, n, k, dtype, 0, dtype, dtype, VX_EPI_STORE,
                        nullptr, 0, st, bias);
    }
    const int64_t tot = m * n;
    dim3 grid((unsigned)vx_cdiv(tot, 256));
    if (dtype == VX_F32)
        hipLaunchKernelGGL(qmm_naive_kernel<VX_F32>, grid, dim3(256), 0, st, x, qweight, scales, biases, bias, y, m, n, k, group_size);
    else if (dtype == VX_F16)
        hipLaunchKernelGGL(qmm_naive_kernel<VX_F16>, grid, dim3(256), 0, st, x, qweight, scales, biases, bias, y, m, n, k, group_size);
    else
        hipLaunchKernelGGL(qmm_naive_kernel<VX_BF16>, grid, dim3(256), 0, st, x, qweight, scales, biases, bias, y, m, n, k, group_size);
    VX_HIP(hipGetLastError());
    return 0;
}

extern "C" int vx_qmm_4bit_ex(const void *x, const uint32_t *qweight, const void *scales,
                              const void *biases, void *y, const void *residual, int64_t m,
                              int64_t n, int64_t k, int64_t group_size, int x_shift,
                              int round_dtype, int y_dtype, int epilogue, void *workspace,
                              size_t workspace_bytes, void *stream) {
    VX_REQUIRE(group_size == 64, "qmm_4bit_ex: group_size must be 64");
    VX_REQUIRE(k % 128 == 0, "qmm_4bit_ex: K must be a multiple of 128");
    if (m == 0 || n == 0) return 0;  // empty tensors may carry null data pointers
    VX_REQUIRE(x && qweight && scales && biases && y, "qmm_4bit_ex: null tensor");
    VX_REQUIRE(epilogue != VX_EPI_RESIDUAL || residual, "qmm_4bit_ex: residual epilogue needs R");
    VX_REQUIRE(fast_ok(VX_F16, k, group_size, x, qweight, scales, biases), "qmm_4bit_ex: misaligned operand");
    return qmm_fast(x, qweight, scales, biases, y, residual, m, n, k, VX_F16, x_shift, round_dtype,
                    y_dtype, epilogue, workspace, workspace_bytes, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// vx_qmm_4bit without allocation.  Its split-K partials live in `scratch`, a
// static device array laid out like a caller workspace (the reserved head,
// then the partials); each GPU holds its own copy until the process ends.
// Kernel arguments take the array's device address from hipGetSymbolAddress,
// resolved once per device on the first call there (the array's name is a
// host-side stand-in, never a device address).
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kNoAllocScratchBytes = VX_QMM_NOALLOC_SCRATCH_BYTES;
static_assert(kNoAllocScratchBytes > kCounterBytes, "the scratch holds the workspace head and the partials");
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

int scratch_address(void **out) {
    static std::mutex mu;
    static std::map<int, void *> per_device;
    int dev = 0;
    VX_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(mu);
    auto it = per_device.find(dev);
    if (it == per_device.end()) {
        void *p = nullptr;
        VX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        VX_REQUIRE(p != nullptr, "qmm_4bit_noalloc: no device address for the static scratch");
        it = per_device.emplace(dev, p).first;
    }
    *out = it->second;
    return 0;
}
}  // namespace

extern "C" int vx_qmm_4bit_noalloc(const void *x, const uint32_t *qweight, const void *scales,
                                   const void *biases, const void *bias, void *y, int64_t m, int64_t n,
                                   int64_t k, int64_t group_size, int dtype, void *stream) {
    // same validation and path choice as vx_qmm_4bit
    VX_REQUIRE(k % 8 == 0, "qmm_4bit: K must be a multiple of 8");
    VX_REQUIRE(group_size != 0 && group_size % 8 == 0 && k % group_size == 0,
               "qmm_4bit: group_size must be a multiple of 8 and divide K");
    VX_REQUIRE(dtype == VX_F32 || dtype == VX_F16 || dtype == VX_BF16, "qmm_4bit: unsupported dtype");
    VX_REQUIRE(m >= 0 && n >= 0, "qmm_4bit: negative shape");
    if (m == 0 || n == 0) return 0;
    VX_REQUIRE(x && qweight && scales && biases && y, "qmm_4bit: null tensor");
    const bool fast = dtype != VX_F32 && fast_ok(dtype, k, group_size, x, qweight, scales, biases) &&
                      m * n < ((int64_t)1 << 31);
    if (!fast)  // the one-thread-per-output kernel needs no scratch
        return vx_qmm_4bit(x, qweight, scales, biases, bias, y, m, n, k, group_size, dtype, stream);
    const size_t need = kCounterBytes + make_plan(m, n, k, VX_EPI_STORE, dtype == VX_F16).partial_bytes;
    if (need > kNoAllocScratchBytes)
        return set_error("qmm_4bit_noalloc: this shape's split-K partials need " + std::to_string(need) +
                         " bytes, above the static scratch of " + std::to_string(kNoAllocScratchBytes) +
                         " bytes (use vx_qmm_4bit_ex with a workspace)");
    void *ws = nullptr;
    VX_TRY(scratch_address(&ws));
    return qmm_fast(x, qweight, scales, biases, y, nullptr, m, n, k, dtype, 0, dtype, dtype, VX_EPI_STORE, ws,
                    kNoAllocScratchBytes, (hipStream_t)stream, bias);
}

extern "C" size_t vx_qmm_workspace_size(int64_t m, int64_t n, int64_t k) {
    size_t a = qmm_workspace_bytes(m, n, k, VX_EPI_STORE, false);
    size_t b = qmm_workspace_bytes(m, n, k, VX_EPI_SWIGLU, false);
    return a > b ? a : b;
}
