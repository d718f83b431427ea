// Shared definitions for the velox_amd HIP library (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/velox_hip.h"

// ---------------------------------------------------------------------------
// error handling: every C-ABI entry returns int (0 ok) and records a message
// readable through vx_last_error() on the calling thread.
// ---------------------------------------------------------------------------
namespace vx {
int set_error(const std::string &msg);
int hip_error(hipError_t e, const char *what);
// A token tree of r nodes (1..64): node 0 is the root (parents[0] < 0) and
// every other node's parent precedes it (0 <= parents[j] < j), so the tree
// has no cycle and every ancestor walk ends at the root.
int check_tree_parents(const int32_t *parents, int64_t r, const char *who);
}  // namespace vx

#define VX_HIP(call)                                            \
    do {                                                        \
        hipError_t _e = (call);                                 \
        if (_e != hipSuccess) return vx::hip_error(_e, #call);  \
    } while (0)

#define VX_REQUIRE(cond, msg)                      \
    do {                                           \
        if (!(cond)) return vx::set_error(msg);    \
    } while (0)

#define VX_TRY(call)                 \
    do {                             \
        int _rc = (call);            \
        if (_rc != 0) return _rc;    \
    } while (0)

// ---------------------------------------------------------------------------
// 16-bit float storage helpers (device side uses the hardware RNE converts).
// ---------------------------------------------------------------------------
typedef _Float16 vx_half;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    // round to nearest even; NaN kept quiet
    // (a select, not a branch: a per-element branch diverges the wave)
    const uint32_t x = __float_as_uint(f);
    const uint32_t rne = (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
    const uint32_t qnan = (x >> 16) | 0x40u;
    return (uint16_t)((x & 0x7fffffffu) > 0x7f800000u ? qnan : rne);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(vx_half, h);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (vx_half)f);
}

// load / store one element of a storage dtype as f32
template <int DT>
__device__ __forceinline__ float ld_elem(const void *p, int64_t i);
template <>
__device__ __forceinline__ float ld_elem<VX_F32>(const void *p, int64_t i) {
    return ((const float *)p)[i];
}
template <>
__device__ __forceinline__ float ld_elem<VX_F16>(const void *p, int64_t i) {
    return f16_bits_to_f32(((const uint16_t *)p)[i]);
}
template <>
__device__ __forceinline__ float ld_elem<VX_BF16>(const void *p, int64_t i) {
    return bf16_bits_to_f32(((const uint16_t *)p)[i]);
}

template <int DT>
__device__ __forceinline__ void st_elem(void *p, int64_t i, float v);
template <>
__device__ __forceinline__ void st_elem<VX_F32>(void *p, int64_t i, float v) {
    ((float *)p)[i] = v;
}
template <>
__device__ __forceinline__ void st_elem<VX_F16>(void *p, int64_t i, float v) {
    ((uint16_t *)p)[i] = f32_to_f16_bits(v);
}
template <>
__device__ __forceinline__ void st_elem<VX_BF16>(void *p, int64_t i, float v) {
    ((uint16_t *)p)[i] = f32_to_bf16_bits(v);
}

// round an f32 value to storage precision DT (returns f32)
template <int DT>
__device__ __forceinline__ float round_to(float v);
template <>
__device__ __forceinline__ float round_to<VX_F32>(float v) { return v; }
template <>
__device__ __forceinline__ float round_to<VX_F16>(float v) { return (float)(vx_half)v; }
template <>
__device__ __forceinline__ float round_to<VX_BF16>(float v) {
    return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

// ---------------------------------------------------------------------------
// Deterministic exp (Cody-Waite reduction + degree-7 Taylor/Horner + 2^k).
// Each step is a single IEEE operation with contraction disabled so the
// result is bit-identical to the host definition used by the acceptance
// tests.  Valid for every input; exp(x) = 0 for x < -87.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ float vx_detexp(float x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x > 88.5f) return __builtin_inff();
    if (x < -87.0f) return 0.0f;
    const float log2e = 1.44269502925872802734375f;
    const float ln2_hi = 0.693145751953125f;
    const float ln2_lo = 1.428606765330187e-06f;
    float kf = __builtin_rintf(x * log2e);
    float r = x - kf * ln2_hi;
    r = r - kf * ln2_lo;
    float p = 1.98412701138295233249664306640625e-04f;
    p = p * r + 1.38888892345130443572998046875e-03f;
    p = p * r + 8.33333376795053482055664062500e-03f;
    p = p * r + 4.16666679084300994873046875000e-02f;
    p = p * r + 1.66666671633720397949218750000e-01f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    int k = (int)kf;
    if (k > 127) {
        p = p * __builtin_bit_cast(float, (uint32_t)(127 + 127) << 23);
        k -= 127;
    }
    return p * __builtin_bit_cast(float, (uint32_t)(k + 127) << 23);
}

// Philox4x32-10 (Salmon et al., SC'11).
__host__ __device__ __forceinline__ void vx_philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c[0] = n0;
        c[1] = n1;
        c[2] = n2;
        c[3] = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}
__host__ __device__ __forceinline__ float vx_u01(uint32_t x) {
    return (float)(x >> 8) * (1.0f / 16777216.0f);
}

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ int64_t vx_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

namespace vx {
int device_cu_count();
// Per-(device, stream) scratch owned by the library for entry points whose
// reference signature carries no workspace.  Grows on demand (never shrinks);
// the first `zero_bytes` of it are kept zero between launches by the kernels
// that use them as counters.
int stream_workspace(hipStream_t s, size_t bytes, void **out);

// The qkv projection's split partials and what finishing them needs (per-head
// norm weights, RoPE tables and positions, KV destinations), handed to the
// attention launcher when it forms q, K and V itself.
struct AttnQkvFuse {
    const float *partial;  // [splits][rows][(h_q + 2 h_kv) * D]
    int splits;
    const uint16_t *qn, *kn, *cos_t, *sin_t;
    const uint32_t *pos, *pages, *slots;
    float eps;
};
}  // namespace vx
