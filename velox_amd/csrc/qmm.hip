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

#include "vx_common.h"

namespace vx {

namespace {

constexpr int kWaves = 4;
constexpr int kChunkGroups = 4;          // groups of 64 staged per LDS chunk
constexpr size_t kCounterBytes = 65536;  // reserved head of the workspace (kept zero)
constexpr size_t kMaxPartialBytes = (size_t)96 << 20;

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
    int col_blocks, m_blocks, per_xcd, total_items;
    int epi, round_dt, y_dt;
    float acc_scale;    // 2^x_shift
    float store_scale;  // 2^-y_shift
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
    float v = round_dt(acc * a.acc_scale, a.round_dt);
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

template <int MT, int NT, bool XBF>
__global__ __launch_bounds__(256) void qmm_int4_kernel(QmmArgs a) {
    __shared__ uint4 xs[kChunkGroups * 2 * MT * 64];
    __shared__ float xsum[XBF ? kChunkGroups * MT * 16 : 1];

    const int bid = blockIdx.x;
    const int item = (bid & 7) * a.per_xcd + (bid >> 3);
    if (item >= a.total_items) return;
    const int cb = item / a.splits;
    const int sp = item - cb * a.splits;
    const int mb = blockIdx.y;
    const int m0 = mb * MT * 16;
    const int g_lo = sp * a.gps;
    const int g_hi = min(a.G, g_lo + a.gps);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kq = lane >> 4;
    const int col0 = cb * (kWaves * NT * 16) + wave * NT * 16 + (lane & 15);
    const int64_t kw = a.K / 8;

    floatx4 acc[MT][NT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[t][nt] = (floatx4){0.f, 0.f, 0.f, 0.f};

    const uint16_t *xh = (const uint16_t *)a.x;
    for (int gc = g_lo; gc < g_hi; gc += kChunkGroups) {
        const int ng = min(kChunkGroups, g_hi - gc);
        // ---- weights + affine params for this chunk (issued before the barrier)
        uint2 wv[kChunkGroups][NT];
        uint2 sv[NT], bv[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int col = min(col0 + nt * 16, a.N - 1);
            const uint32_t *wr = a.w + (int64_t)col * kw + (int64_t)gc * 8 + 2 * kq;
#pragma unroll
            for (int gg = 0; gg < kChunkGroups; gg++)
                wv[gg][nt] = gg < ng ? *(const uint2 *)(wr + gg * 8) : make_uint2(0u, 0u);
            sv[nt] = *(const uint2 *)(a.s + (int64_t)col * a.G + gc);
            bv[nt] = *(const uint2 *)(a.b + (int64_t)col * a.G + gc);
        }
        __syncthreads();  // previous chunk's fragments fully consumed
        // ---- stage activations in fragment order
        for (int u = tid; u < ng * 2 * MT * 64; u += 256) {
            const int l = u & 63;
            int r = u >> 6;
            const int t = r % MT;
            r /= MT;
            const int s = r & 1;
            const int gg = r >> 1;
            const int row = m0 + t * 16 + (l & 15);
            const int kk = (gc + gg) * 64 + 8 * (2 * (l >> 4) + s);
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (row < a.M) v = *(const uint4 *)(xh + (int64_t)row * a.K + kk);
            xs[u] = permute_k8(v);
        }
        if (XBF) {
            for (int idx = tid; idx < ng * MT * 16; idx += 256) {
                const int gg = idx / (MT * 16);
                const int rr = idx - gg * MT * 16;
                const int row = m0 + rr;
                float sum = 0.f;
                if (row < a.M) {
                    const uint16_t *xr = xh + (int64_t)row * a.K + (gc + gg) * 64;
                    for (int e = 0; e < 64; e++) sum += bf16_bits_to_f32(xr[e]);
                }
                xsum[gg * MT * 16 + rr] = sum;
            }
        }
        __syncthreads();
        // ---- MFMA over the chunk
#pragma unroll
        for (int gg = 0; gg < kChunkGroups; gg++) {
            if (gg >= ng) break;
            if constexpr (!XBF) {
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    half8_t af[MT];
#pragma unroll
                    for (int t = 0; t < MT; t++)
                        af[t] = __builtin_bit_cast(half8_t, xs[((gg * 2 + s) * MT + t) * 64 + lane]);
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        const uint32_t word = s == 0 ? wv[gg][nt].x : wv[gg][nt].y;
                        const uint32_t sbits = gg < 2 ? sv[nt].x : sv[nt].y;
                        const uint32_t bbits = gg < 2 ? bv[nt].x : bv[nt].y;
                        const uint16_t sh = (gg & 1) ? (uint16_t)(sbits >> 16) : (uint16_t)sbits;
                        const uint16_t bh = (gg & 1) ? (uint16_t)(bbits >> 16) : (uint16_t)bbits;
                        const vx_half sc = __builtin_bit_cast(vx_half, sh);
                        const vx_half bi = __builtin_bit_cast(vx_half, bh);
                        const half8_t bf = dequant_f16(word, (half2_t){sc, sc}, (half2_t){bi, bi});
#pragma unroll
                        for (int t = 0; t < MT; t++)
                            acc[t][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], bf, acc[t][nt], 0, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const uint32_t sbits = gg < 2 ? sv[nt].x : sv[nt].y;
                    const uint32_t bbits = gg < 2 ? bv[nt].x : bv[nt].y;
                    const float sc = bf16_bits_to_f32((gg & 1) ? (uint16_t)(sbits >> 16) : (uint16_t)sbits);
                    const float bi = bf16_bits_to_f32((gg & 1) ? (uint16_t)(bbits >> 16) : (uint16_t)bbits);
                    const float boff = bi - 128.0f * sc;
                    const bf16x8_t b0 = codes_bf16(wv[gg][nt].x);
                    const bf16x8_t b1 = codes_bf16(wv[gg][nt].y);
#pragma unroll
                    for (int t = 0; t < MT; t++) {
                        floatx4 tmp = {0.f, 0.f, 0.f, 0.f};
                        tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8_t, xs[((gg * 2 + 0) * MT + t) * 64 + lane]), b0, tmp, 0, 0, 0);
                        tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8_t, xs[((gg * 2 + 1) * MT + t) * 64 + lane]), b1, tmp, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const float xsr = xsum[gg * MT * 16 + t * 16 + 4 * kq + r];
                            acc[t][nt][r] += sc * tmp[r] + boff * xsr;
                        }
                    }
                }
            }
        }
    }

    // ---- split-K: publish the partial tile; qmm_reduce_kernel finishes
    if (a.splits > 1) {
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

    // ---- epilogue
    if (a.epi == VX_EPI_SWIGLU) {
        // tiles come in (gate, up) pairs: global tile 2f = gate rows, 2f+1 = up rows
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int nt = 0; nt + 1 < NT; nt += 2) {
                const int gtile = (col0 - (lane & 15)) / 16 + nt;
                const int f = (gtile / 2) * 16 + (lane & 15);
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

template <int DT>
__global__ void add_bias_kernel(void *y, const void *bias, int64_t m, int64_t n) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= m * n) return;
    st_elem<DT>(y, idx, ld_elem<DT>(y, idx) + ld_elem<DT>(bias, idx % n));
}

struct Plan {
    int MT, NT, splits, gps, col_blocks, m_blocks, per_xcd, total_items;
    size_t partial_bytes;
};

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

Plan make_plan(int64_t M, int64_t N, int64_t K, int epi) {
    Plan p{};
    const int64_t mrows = std::min<int64_t>(M, 80);
    p.MT = (int)std::max<int64_t>(1, vx_cdiv(mrows, 16));
    p.m_blocks = (int)vx_cdiv(M, p.MT * 16);
    int nt = p.MT >= 3 ? 4 : (p.MT == 2 ? 2 : 1);
    if (epi == VX_EPI_SWIGLU) nt = std::max(nt, 2);
    const int G = (int)(K / 64);
    const int cus = device_cu_count();
    const int target = 2 * cus;
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
    p.total_items = p.col_blocks * splits;
    p.per_xcd = (int)vx_cdiv(p.total_items, 8);
    p.partial_bytes = splits > 1 ? (size_t)splits * M * N * 4 : 0;
    return p;
}

template <int MT, int NT, bool XBF>
void launch_fast(const QmmArgs &a, const Plan &p, hipStream_t st) {
    dim3 grid(p.per_xcd * 8, p.m_blocks);
    hipLaunchKernelGGL((qmm_int4_kernel<MT, NT, XBF>), grid, dim3(256), 0, st, a);
    if (p.splits > 1) {
        const int64_t outs = (int64_t)a.M * (a.epi == VX_EPI_SWIGLU ? a.N / 2 : a.N);
        hipLaunchKernelGGL(qmm_reduce_kernel, dim3((unsigned)vx_cdiv(outs, 256)), dim3(256), 0, st, a);
    }
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

bool fast_ok(int64_t K, int64_t gs, const void *x, const void *w, const void *s, const void *b) {
    return gs == 64 && K % 256 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 8) == 0 &&
           ((uintptr_t)s % 8) == 0 && ((uintptr_t)b % 8) == 0;
}

}  // namespace

size_t qmm_workspace_bytes(int64_t m, int64_t n, int64_t k, int epi) {
    if (k % 256 != 0) return kCounterBytes;
    Plan p = make_plan(m, n, k, epi);
    return kCounterBytes + p.partial_bytes;
}

int qmm_launch(const void *x, const uint32_t *w, const void *s, const void *b, void *y,
               const void *resid, int64_t M, int64_t N, int64_t K, int x_dt, int x_shift,
               int y_shift, int round_dt, int y_dt, int epi, void *workspace, size_t ws_bytes,
               hipStream_t st) {
    Plan p = make_plan(M, N, K, epi);
    if (epi == VX_EPI_SWIGLU && (N % 32 != 0 || p.NT % 2 != 0))
        return set_error("qmm swiglu: N must be a multiple of 32 with paired tiles");
    void *ws = workspace;
    if (p.splits > 1) {
        if (!ws) {
            VX_TRY(stream_workspace(st, kCounterBytes + p.partial_bytes, &ws));
        } else if (ws_bytes < kCounterBytes + p.partial_bytes) {
            return set_error("qmm: workspace too small (see vx_qmm_workspace_size)");
        }
    }
    QmmArgs a;
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
    a.col_blocks = p.col_blocks;
    a.m_blocks = p.m_blocks;
    a.per_xcd = p.per_xcd;
    a.total_items = p.total_items;
    a.epi = epi;
    a.round_dt = round_dt;
    a.y_dt = y_dt;
    a.acc_scale = ldexpf(1.0f, x_shift);
    a.store_scale = ldexpf(1.0f, -y_shift);
    int rc = x_dt == VX_BF16 ? dispatch_fast<true>(a, p, st) : dispatch_fast<false>(a, p, st);
    if (rc) return rc;
    VX_HIP(hipGetLastError());
    return 0;
}

int qmm_fast(const void *x, const uint32_t *w, const void *s, const void *b, void *y,
             const void *resid, int64_t M, int64_t N, int64_t K, int x_dt, int x_shift,
             int round_dt, int y_dt, int epi, void *workspace, size_t ws_bytes, hipStream_t st) {
    return qmm_launch(x, w, s, b, y, resid, M, N, K, x_dt, x_shift, 0, round_dt, y_dt, epi, workspace,
                      ws_bytes, st);
}

// f16 activations (optionally stored as X * 2^-x_shift); the result is scaled
// by 2^x_shift, rounded to round_dt, and stored as value * 2^-y_shift.
int qmm_fast_scaled(const void *x, const uint32_t *w, const void *s, const void *b, void *y,
                    const void *resid, int64_t M, int64_t N, int64_t K, int x_shift, int y_shift,
                    int round_dt, int y_dt, int epi, void *workspace, size_t ws_bytes, hipStream_t st) {
    return qmm_launch(x, w, s, b, y, resid, M, N, K, VX_F16, x_shift, y_shift, round_dt, y_dt, epi,
                      workspace, ws_bytes, st);
}

}  // namespace vx

using namespace vx;

extern "C" int vx_qmm_4bit(const void *x, const uint32_t *qweight, const void *scales,
                           const void *biases, const void *bias, void *y, int64_t m, int64_t n,
                           int64_t k, int64_t group_size, int dtype, void *stream) {
    // validation mirrors metal_kernels.rs:2082-2130
    VX_REQUIRE(k % 8 == 0, "qmm_4bit: K must be a multiple of 8");
    VX_REQUIRE(group_size != 0 && group_size % 8 == 0 && k % group_size == 0,
               "qmm_4bit: group_size must be a multiple of 8 and divide K");
    VX_REQUIRE(dtype == VX_F32 || dtype == VX_F16 || dtype == VX_BF16, "qmm_4bit: unsupported dtype");
    VX_REQUIRE(m >= 0 && n >= 0, "qmm_4bit: negative shape");
    VX_REQUIRE(x && qweight && scales && biases && y, "qmm_4bit: null tensor");
    if (m == 0 || n == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    if (dtype != VX_F32 && fast_ok(k, group_size, x, qweight, scales, biases) && m * n < ((int64_t)1 << 31)) {
        VX_TRY(qmm_fast(x, qweight, scales, biases, y, nullptr, m, n, k, dtype, 0, dtype, dtype,
                        VX_EPI_STORE, nullptr, 0, st));
        if (bias) {
            const int64_t tot = m * n;
            if (dtype == VX_BF16)
                hipLaunchKernelGGL(add_bias_kernel<VX_BF16>, dim3((unsigned)vx_cdiv(tot, 256)), dim3(256), 0, st, y, bias, m, n);
            else
                hipLaunchKernelGGL(add_bias_kernel<VX_F16>, dim3((unsigned)vx_cdiv(tot, 256)), dim3(256), 0, st, y, bias, m, n);
            VX_HIP(hipGetLastError());
        }
        return 0;
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
    VX_REQUIRE(k % 256 == 0, "qmm_4bit_ex: K must be a multiple of 256");
    VX_REQUIRE(x && qweight && scales && biases && y, "qmm_4bit_ex: null tensor");
    VX_REQUIRE(epilogue != VX_EPI_RESIDUAL || residual, "qmm_4bit_ex: residual epilogue needs R");
    VX_REQUIRE(fast_ok(k, group_size, x, qweight, scales, biases), "qmm_4bit_ex: misaligned operand");
    if (m == 0 || n == 0) return 0;
    return qmm_fast(x, qweight, scales, biases, y, residual, m, n, k, VX_F16, x_shift, round_dtype,
                    y_dtype, epilogue, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" size_t vx_qmm_workspace_size(int64_t m, int64_t n, int64_t k) {
    size_t a = qmm_workspace_bytes(m, n, k, VX_EPI_STORE);
    size_t b = qmm_workspace_bytes(m, n, k, VX_EPI_SWIGLU);
    return a > b ? a : b;
}
