// Engine level of the verify path: PagedKvCache (reference src/paged/pages.rs),
// PagedQwen3 forward / forward_all (src/paged/qwen3.rs:943-1037) and
// SpecEngine prefill / step / free (src/paged/spec.rs), hosted in C++ over the
// gfx950 kernels.
//
// Numerics follow the reference's bf16 model (vb.dtype() == BF16, as in
// tests/spec_decode.rs:162): every tensor value is rounded to bf16 at the same
// points as candle's ops.  GEMM inputs, Q and the KV pages are stored as f16,
// which holds each of those bf16 values exactly (|v| < 65504), so the MFMA
// f16 path computes on the reference's values.  The MLP product uses a 2^-8
// storage scale (exact) to keep |v| < 65504 in f16.
//
// One round (spec.rs:186-316) on the device:
//   host: grow block tables (all-or-nothing page allocation), build every
//         forward's row metadata and upload it in one copy;
//   D draft forwards over the batch (argmax -> next draft input on device);
//   one verify forward over batch x (D+1) rows; one acceptance launch;
//   one device->host copy of (accepted, committed tokens, candidates).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "vx_common.h"

namespace vx {

// ---------------------------------------------------------------------------
// library state
// ---------------------------------------------------------------------------
static thread_local std::string g_err;
int set_error(const std::string &msg) {
    g_err = msg;
    return -1;
}
int hip_error(hipError_t e, const char *what) {
    g_err = std::string(what) + ": " + hipGetErrorString(e);
    return -2;
}

int check_tree_parents(const int32_t *parents, int64_t r, const char *who) {
    const std::string w(who);
    VX_REQUIRE(r >= 1 && r <= 64, w + ": a tree holds 1..64 nodes");
    VX_REQUIRE(parents && parents[0] < 0, w + ": node 0 must be the root");
    for (int64_t j = 1; j < r; j++)
        VX_REQUIRE(parents[j] >= 0 && parents[j] < j, w + ": parents[j] must precede j");
    return 0;
}

int device_cu_count() {
    static std::mutex mu;
    static std::map<int, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
    cache[dev] = cus;
    return cus;
}

// Library-owned workspace per (device, stream) for the entry points called
// without one.  It grows geometrically; a superseded buffer is never freed
// while the library is loaded, because another host thread on the same
// stream may still be queueing kernels that read it (at most the final size
// again is held in retired buffers).
int stream_workspace(hipStream_t s, size_t bytes, void **out) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, std::pair<void *, size_t>> ws;
    static std::vector<void *> retired;
    int dev = 0;
    VX_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(mu);
    auto &e = ws[{dev, s}];
    if (e.first && e.second >= bytes) {
        *out = e.first;
        return 0;
    }
    size_t sz = std::max(bytes, e.second * 2);
    sz = (sz + 4095) & ~(size_t)4095;
    void *p = nullptr;
    VX_HIP(hipMalloc(&p, sz));
    VX_HIP(hipMemsetAsync(p, 0, sz, s));
    if (e.first) retired.push_back(e.first);
    e.first = p;
    e.second = sz;
    *out = p;
    return 0;
}

// kernels in the other translation units
size_t qmm_packed_bytes(int64_t n, int64_t k);
int qmm_pack(const uint32_t *w, const void *s, const void *b, void *out, int64_t N, int64_t K, hipStream_t st);
int qmm_packed(const void *x, const void *packed, void *y, const void *resid, int64_t M, int64_t N, int64_t K,
               int x_shift, int y_shift, int round_dt, int y_dt, int epi, void *workspace, size_t ws_bytes,
               hipStream_t st);
size_t qmm_workspace_bytes(int64_t m, int64_t n, int64_t k, int epi, bool packed);
size_t attn_workspace_bound(int64_t n_seqs, int64_t h_kv, int64_t max_rows, int64_t G, int64_t D, int64_t max_kv);
int paged_attention_launch(const void *q, const void *k_pool, const void *v_pool, const uint32_t *bt,
                           const uint32_t *cu, const uint32_t *kvo, const uint64_t *tmask, void *out,
                           int mode, int64_t total_q, int64_t n_seqs, int64_t max_rows,
                           int64_t max_blocks, int64_t num_pages, int64_t h_q, int64_t h_kv,
                           int64_t D, int64_t ps, float scale, uint32_t window, int dtype,
                           void *workspace, size_t ws_bytes, int64_t max_kv, hipStream_t st,
                           int out_bf16_round, const AttnQkvFuse *fuse);
size_t accept_workspace_bytes(int64_t rows, int64_t vocab);
size_t stochastic_workspace_bytes(int64_t rows, int64_t vocab);
int argmax_accept_launch(const void *logits, int ldt, int64_t rows, int64_t vocab, int mode,
                         int rows_per_group, const uint32_t *cand, int k, int32_t *accepted,
                         uint32_t *tokens, int32_t *path, const int32_t *parents, uint32_t *argmax_out,
                         uint32_t *next_ids, int64_t next_stride, void *ws, size_t ws_bytes,
                         hipStream_t st);
int sample_rows_launch(const void *logits, int ldt, const float *uni, int64_t ustride, uint32_t *out,
                       int64_t rows, int64_t vocab, float temperature, uint32_t *next_ids,
                       int64_t next_stride, void *ws, size_t ws_bytes, hipStream_t st);
int stochastic_accept_launch(const void *tl, const void *dl, int ldt, const uint32_t *cand,
                             const float *uni, int32_t *accepted, uint32_t *tokens, int64_t batch,
                             int64_t k, int64_t vocab, float temperature, bool draft_step_major, void *ws,
                             size_t ws_bytes, hipStream_t st);
int embed_rmsnorm_launch(const uint32_t *ids, int64_t ids_stride, const uint16_t *embed, int64_t vocab,
                         const uint16_t *w, uint16_t *h, uint16_t *y, int64_t rows, int64_t H, float eps, int out_dt,
                         hipStream_t st);
int rmsnorm_launch(const uint16_t *x, const uint16_t *w, uint16_t *y, const uint32_t *row_idx,
                   int64_t rows, int64_t H, float eps, int out_dt, hipStream_t st);
int qkv_partial_rope_scatter_launch(const float *partial, int splits, const uint16_t *qn, const uint16_t *kn,
                                    const uint16_t *cos_t, const uint16_t *sin_t, const uint32_t *pos,
                                    const uint32_t *pages, const uint32_t *slots, uint16_t *qout, uint16_t *kp,
                                    uint16_t *vp, int64_t rows, int HQ, int HK, int D, int ps, float eps, int kv_dt,
                                    hipStream_t st);
int residual_rmsnorm_launch(const float *partial, int splits, float acc_scale, uint16_t *h, const uint16_t *ln,
                            uint16_t *y, int64_t rows, int64_t H, float eps, int out_dt, hipStream_t st);
bool qmm_packed_argmax_ok(int64_t M, int64_t N, int64_t K);
int qmm_packed_argmax(const void *x, const void *packed, void *y, int64_t M, int64_t N, int64_t K, int round_dt,
                      int y_dt, float *amax_v, uint32_t *amax_i, void *workspace, size_t ws_bytes, hipStream_t st);
int argmax_accept_partials_launch(const float *pv, const uint32_t *pi, int n_chunks, int64_t rows, int mode,
                                  int rows_per_group, const uint32_t *cand, int k, int32_t *accepted,
                                  uint32_t *tokens, uint32_t *next_ids, int64_t next_stride, hipStream_t st);
size_t qmm_partial_ws_bytes(int64_t M, int64_t N, int64_t K);
int qmm_packed_partial(const void *x, const void *packed, int64_t M, int64_t N, int64_t K, void *workspace,
                       size_t ws_bytes, int *splits, const float **partial, hipStream_t st);

// ---------------------------------------------------------------------------
// host-side 16-bit conversions (RNE), identical to the device converts
// ---------------------------------------------------------------------------
static inline float h2f(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            float v = (float)m * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
static inline uint16_t f2bf(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}
static inline float bf2f(uint16_t h) {
    uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}
static inline uint16_t f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x33000000u) return (uint16_t)sign;
    const int e = (int)(ax >> 23) - 127;
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    if (e >= -14) {
        uint32_t h = ((uint32_t)(e + 15) << 10) | ((mant >> 13) & 0x3ffu);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    const int s = -e - 1;
    uint32_t h = mant >> s;
    const uint32_t rem = mant & ((1u << s) - 1u), half = 1u << (s - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}
// f16 -> bf16 value (candle VarBuilder to_dtype), kept in an f16 carrier
static inline uint16_t f16_as_bf16_carrier(uint16_t h) { return f2h(bf2f(f2bf(h2f(h)))); }
static inline uint16_t f16_to_bf16_bits(uint16_t h) { return f2bf(h2f(h)); }

}  // namespace vx

using namespace vx;

// ===========================================================================
// pages (pages.rs)
// ===========================================================================
struct vx_pages {
    int64_t layers = 0, kv_heads = 0, head_dim = 0, page_size = 0, num_pages = 0;
    int dtype = VX_F16;
    int device = 0;
    void *base = nullptr;
    size_t pool_bytes = 0;  // per (layer, K|V)
    std::vector<uint32_t> free_list;
    std::vector<uint32_t> refcount;
    std::mutex mu;
};

extern "C" int vx_pages_create(int64_t layers, int64_t kv_heads, int64_t head_dim, int64_t page_size,
                               int64_t num_pages, int kv_dtype, vx_pages **out) {
    VX_REQUIRE(out, "pages: null out");
    VX_REQUIRE(layers > 0 && num_pages > 0, "PagedKvCache must have >=1 layer and >=1 page");
    VX_REQUIRE(num_pages <= (int64_t)UINT32_MAX, "num_pages exceeds u32 range");
    VX_REQUIRE(kv_dtype == VX_F16 || kv_dtype == VX_BF16, "pages: kv dtype must be f16 or bf16");
    auto p = std::make_unique<vx_pages>();
    p->layers = layers;
    p->kv_heads = kv_heads;
    p->head_dim = head_dim;
    p->page_size = page_size;
    p->num_pages = num_pages;
    p->dtype = kv_dtype;
    VX_HIP(hipGetDevice(&p->device));
    p->pool_bytes = (size_t)num_pages * kv_heads * page_size * head_dim * 2;
    const size_t total = p->pool_bytes * layers * 2;
    VX_HIP(hipMalloc(&p->base, total));
    VX_HIP(hipMemset(p->base, 0, total));
    p->free_list.resize(num_pages);
    for (int64_t i = 0; i < num_pages; i++) p->free_list[i] = (uint32_t)(num_pages - 1 - i);
    p->refcount.assign(num_pages, 0);
    *out = p.release();
    return 0;
}

extern "C" void vx_pages_destroy(vx_pages *p) {
    if (!p) return;
    if (p->base) (void)hipFree(p->base);
    delete p;
}

extern "C" int vx_pages_alloc(vx_pages *p, int64_t n, uint32_t *out_pages) {
    VX_REQUIRE(p && (out_pages || n == 0), "pages: null argument");
    std::lock_guard<std::mutex> lk(p->mu);
    if ((int64_t)p->free_list.size() < n) return set_error("alloc: not enough free pages");
    for (int64_t i = 0; i < n; i++) {
        const uint32_t pg = p->free_list.back();
        p->free_list.pop_back();
        p->refcount[pg] = 1;
        out_pages[i] = pg;
    }
    return 0;
}

extern "C" void vx_pages_incref(vx_pages *p, const uint32_t *pages, int64_t n) {
    if (!p) return;
    std::lock_guard<std::mutex> lk(p->mu);
    for (int64_t i = 0; i < n; i++)
        if ((int64_t)pages[i] < p->num_pages && p->refcount[pages[i]] >= 1) p->refcount[pages[i]]++;
}

extern "C" void vx_pages_free(vx_pages *p, const uint32_t *pages, int64_t n) {
    if (!p) return;
    std::lock_guard<std::mutex> lk(p->mu);
    for (int64_t i = 0; i < n; i++) {
        const uint32_t pg = pages[i];
        if ((int64_t)pg >= p->num_pages || p->refcount[pg] == 0) continue;
        if (--p->refcount[pg] == 0) p->free_list.push_back(pg);
    }
}

extern "C" int64_t vx_pages_num_free(const vx_pages *p) {
    if (!p) return 0;
    std::lock_guard<std::mutex> lk(const_cast<vx_pages *>(p)->mu);
    return (int64_t)p->free_list.size();
}

extern "C" uint32_t vx_pages_refcount(const vx_pages *p, uint32_t page) {
    if (!p || (int64_t)page >= p->num_pages) return 0;
    std::lock_guard<std::mutex> lk(const_cast<vx_pages *>(p)->mu);
    return p->refcount[page];
}

extern "C" void *vx_pages_pool(vx_pages *p, int64_t layer, int kv) {
    if (!p || layer < 0 || layer >= p->layers) return nullptr;
    return (char *)p->base + (size_t)(layer * 2 + (kv ? 1 : 0)) * p->pool_bytes;
}

namespace {

// Tree-path KV compaction: one workgroup per (sequence, layer x {K, V}, kv
// head).  The accepted path's rows (node path[d] at position kv_offset +
// path[d], d = 1..A) are first read into LDS, then written at kv_offset + d,
// so every destination receives its source's value from before the move
// (path[d] >= d: a destination never precedes a source still to be read in
// sequential order either).  Rows move as raw 32-bit words.
__global__ __launch_bounds__(256) void kv_compact_path_kernel(uint8_t *base, size_t pool_bytes, const uint32_t *bt,
                                                              int max_blocks, const uint32_t *kv_offsets,
                                                              const int32_t *accepted, const int32_t *path, int r,
                                                              int kv_heads, int page_size, int num_pages,
                                                              int row_words) {
    extern __shared__ uint32_t rows[];
    const int b = blockIdx.x;
    const int pool = blockIdx.y;  // layer * 2 + (K|V)
    const int h = blockIdx.z;
    const int A = min(max(accepted[b], 0), r - 1);
    const int64_t kv0 = kv_offsets[b];
    const uint32_t *btr = bt + (int64_t)b * max_blocks;
    uint32_t *pw = (uint32_t *)(base + (size_t)pool * pool_bytes);
    auto row_at = [&](int64_t pos) -> int64_t {  // word offset of (pos, head h)
        const int blk = (int)min<int64_t>(pos / page_size, max_blocks - 1);
        const int64_t page = min<int64_t>(btr[blk], num_pages - 1);
        return ((page * kv_heads + h) * page_size + pos % page_size) * row_words;
    };
    for (int i = threadIdx.x; i < A * row_words; i += blockDim.x) {
        const int d = 1 + i / row_words;
        const int src = min(max(path[(int64_t)b * r + d], 0), r - 1);
        rows[i] = pw[row_at(kv0 + src) + i % row_words];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < A * row_words; i += blockDim.x) {
        const int d = 1 + i / row_words;
        pw[row_at(kv0 + d) + i % row_words] = rows[i];
    }
}

}  // namespace

extern "C" int vx_kv_compact_path(vx_pages *p, const uint32_t *block_tables, int64_t max_blocks,
                                  const uint32_t *kv_offsets, const int32_t *accepted, const int32_t *path,
                                  int64_t n_seqs, int64_t r, void *stream) {
    VX_REQUIRE(p, "kv_compact_path: null pages");
    VX_REQUIRE(r >= 1 && r <= 64, "kv_compact_path: tree of 1..64 nodes");
    VX_REQUIRE(max_blocks >= 1, "kv_compact_path: empty block table");
    if (n_seqs == 0) return 0;
    VX_REQUIRE(block_tables && kv_offsets && accepted && path, "kv_compact_path: null tensor");
    const int row_words = (int)(p->head_dim * 2 / 4);
    VX_REQUIRE(p->head_dim % 2 == 0, "kv_compact_path: head_dim must be even");
    const size_t lds = (size_t)(r - 1) * row_words * 4;
    if (r == 1) return 0;
    hipLaunchKernelGGL(kv_compact_path_kernel, dim3((unsigned)n_seqs, (unsigned)(p->layers * 2), (unsigned)p->kv_heads),
                       dim3(256), lds, (hipStream_t)stream, (uint8_t *)p->base, p->pool_bytes, block_tables,
                       (int)max_blocks, kv_offsets, accepted, path, (int)r, (int)p->kv_heads, (int)p->page_size,
                       (int)p->num_pages, row_words);
    VX_HIP(hipGetLastError());
    return 0;
}

// ===========================================================================
// model (qwen3.rs)
// ===========================================================================
namespace {

struct QLinDev {
    void *packed = nullptr;  // packed int4 blocks; affine params as f16 carriers of bf16 values
    int64_t n = 0, k = 0;
};

struct LayerDev {
    uint16_t *ln1, *ln2, *qn, *kn;  // bf16
    QLinDev qkv, o, gu, down;
};

struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
    int ensure(size_t bytes) {
        if (n >= bytes) return 0;
        if (p) VX_HIP(hipFree(p));
        p = nullptr;
        n = 0;
        VX_HIP(hipMalloc(&p, bytes));
        n = bytes;
        return 0;
    }
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

// Row metadata of one forward, built on the host and uploaded as one blob.
struct Meta {
    int64_t rows = 0, n_seqs = 0, max_blocks = 1, max_rows = 1, max_kv = 1;
    bool tree = false;
    bool one_row = false;  // every sequence brings exactly one row (row s is its last row)
    // offsets (bytes) inside the blob
    size_t o_pos, o_page, o_slot, o_cu, o_kvo, o_bt, o_mask, o_last, size;
};

constexpr int kMlpShift = 8;  // MLP product stored as v * 2^-8 in f16

// Opt-in per-kernel timing with HIP events recorded on the launch stream.
enum ProfClass { PC_QMM = 0, PC_ATTN = 1, PC_OTHER = 2, PC_N = 3 };
struct Prof {
    bool on = false;
    std::vector<hipEvent_t> pool;
    size_t used = 0;
    struct Rec {
        hipEvent_t a, b;
        int cls;
        double bytes;
    };
    std::vector<Rec> recs;
    hipEvent_t next() {
        if (used == pool.size()) {
            hipEvent_t e;
            (void)hipEventCreate(&e);
            pool.push_back(e);
        }
        return pool[used++];
    }
    void reset() {
        used = 0;
        recs.clear();
    }
    ~Prof() {
        for (hipEvent_t e : pool) (void)hipEventDestroy(e);
    }
};

struct ProfScope {
    Prof *p;
    hipStream_t st;
    Prof::Rec r{};
    ProfScope(Prof *p_, hipStream_t st_, int cls, double bytes) : p(p_), st(st_) {
        if (!p || !p->on) return;
        r.a = p->next();
        r.b = p->next();
        r.cls = cls;
        r.bytes = bytes;
        (void)hipEventRecord(r.a, st);
    }
    ~ProfScope() {
        if (!p || !p->on) return;
        (void)hipEventRecord(r.b, st);
        p->recs.push_back(r);
    }
};

// algorithmic bytes of one int4 GEMM launch: packed weights + f16 affine
// params (0.5625 B/weight), X read once, Y written once (+ R read)
double qmm_bytes(int64_t M, int64_t N, int64_t K, bool resid) {
    return 0.5625 * (double)N * K + 2.0 * M * K + 2.0 * M * N * (resid ? 2 : 1);
}

}  // namespace

struct vx_model {
    vx_qwen3_config cfg{};
    int64_t L = 0;
    int device = 0;
    uint16_t *embed = nullptr;  // bf16 [V, H]
    std::vector<LayerDev> layers;
    uint16_t *norm = nullptr;
    QLinDev lm;
    uint16_t *cos_t = nullptr, *sin_t = nullptr;  // bf16 [max_pos, D/2]
    std::vector<void *> allocs;
    // activations
    DevBuf h, xn, q, attn, act, ids, meta, ws;
    int64_t cap_rows = 0;
    ~vx_model() {
        for (void *p : allocs) (void)hipFree(p);
    }
};

namespace {

int dev_upload(vx_model *m, const void *src, size_t bytes, void **dst) {
    void *p = nullptr;
    VX_HIP(hipMalloc(&p, std::max<size_t>(bytes, 16)));
    m->allocs.push_back(p);
    VX_HIP(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice));
    *dst = p;
    return 0;
}

// Concatenate linears row-wise (optionally interleaving 16-row blocks of two
// linears) and convert the affine params to bf16 values in f16 carriers.
int upload_qlin(vx_model *m, const std::vector<const vx_qlinear_host *> &parts,
                const std::vector<int64_t> &ns, int64_t k, bool interleave16, QLinDev *out) {
    const int64_t g = k / 64, kw = k / 8;
    int64_t n = 0;
    for (int64_t x : ns) n += x;
    std::vector<uint32_t> w((size_t)(n * kw));
    std::vector<uint16_t> s((size_t)(n * g)), b((size_t)(n * g));
    auto put_row = [&](int64_t dst, const vx_qlinear_host *src, int64_t r) {
        memcpy(&w[dst * kw], src->qweight + r * kw, kw * 4);
        for (int64_t j = 0; j < g; j++) {
            s[dst * g + j] = f16_as_bf16_carrier(src->scales[r * g + j]);
            b[dst * g + j] = f16_as_bf16_carrier(src->biases[r * g + j]);
        }
    };
    if (interleave16) {
        const int64_t f = ns[0];
        if (ns.size() != 2 || ns[1] != f || f % 16) return set_error("gate/up interleave needs equal N % 16 == 0");
        for (int64_t blk = 0; blk < f / 16; blk++)
            for (int64_t i = 0; i < 16; i++) {
                put_row(blk * 32 + i, parts[0], blk * 16 + i);
                put_row(blk * 32 + 16 + i, parts[1], blk * 16 + i);
            }
    } else {
        int64_t row = 0;
        for (size_t p = 0; p < parts.size(); p++)
            for (int64_t r = 0; r < ns[p]; r++) put_row(row++, parts[p], r);
    }
    out->n = n;
    out->k = k;
    // stage the row-major tensors, pack on the device, drop the staging copies
    void *tw = nullptr, *ts = nullptr, *tb = nullptr, *pk = nullptr;
    auto release = [&]() {
        (void)hipFree(tw);
        (void)hipFree(ts);
        (void)hipFree(tb);
    };
    if (hipMalloc(&tw, w.size() * 4) != hipSuccess || hipMalloc(&ts, s.size() * 2) != hipSuccess ||
        hipMalloc(&tb, b.size() * 2) != hipSuccess || hipMalloc(&pk, qmm_packed_bytes(n, k)) != hipSuccess) {
        release();
        (void)hipFree(pk);
        return set_error("model: out of device memory for weights");
    }
    m->allocs.push_back(pk);
    int rc = 0;
    if (hipMemcpy(tw, w.data(), w.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(ts, s.data(), s.size() * 2, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(tb, b.data(), b.size() * 2, hipMemcpyHostToDevice) != hipSuccess)
        rc = set_error("model: weight upload failed");
    if (!rc) rc = qmm_pack((const uint32_t *)tw, ts, tb, pk, n, k, nullptr);
    if (!rc && hipDeviceSynchronize() != hipSuccess) rc = set_error("model: weight packing failed");
    release();
    out->packed = pk;
    return rc;
}

int upload_bf16(vx_model *m, const uint16_t *f16, int64_t n, uint16_t **out) {
    std::vector<uint16_t> t((size_t)n);
    for (int64_t i = 0; i < n; i++) t[i] = f16_to_bf16_bits(f16[i]);
    return dev_upload(m, t.data(), t.size() * 2, (void **)out);
}

}  // namespace

extern "C" int vx_model_create(const vx_qwen3_config *cfg, const vx_weights_host *w, int64_t n_layers,
                               vx_model **out) {
    VX_REQUIRE(cfg && w && out, "model: null argument");
    const int64_t L = n_layers > 0 ? std::min(n_layers, cfg->layers) : cfg->layers;
    const int64_t H = cfg->hidden, F = cfg->inter, D = cfg->head_dim, HQ = cfg->n_heads, HK = cfg->n_kv_heads;
    VX_REQUIRE(cfg->group_size == 64, "model: only MLX int4 group_size 64 is supported");
    VX_REQUIRE(H % 256 == 0 && F % 256 == 0 && (HQ * D) % 256 == 0, "model: hidden/inter/heads*head_dim must be multiples of 256");
    VX_REQUIRE(HK > 0 && HQ % HK == 0, "model: n_heads must be divisible by n_kv_heads");
    VX_REQUIRE(H <= 8192, "model: hidden size above 8192 is not supported");
    VX_REQUIRE(D % 32 == 0 && D <= 256, "model: head_dim must be a multiple of 32 and <= 256");
    VX_REQUIRE(F % 16 == 0, "model: intermediate size must be a multiple of 16");
    VX_REQUIRE(cfg->vocab % 32 == 0, "model: vocab must be a multiple of 32");
    auto m = std::make_unique<vx_model>();
    m->cfg = *cfg;
    m->L = L;
    VX_HIP(hipGetDevice(&m->device));
    VX_TRY(upload_bf16(m.get(), w->embed, cfg->vocab * H, &m->embed));
    VX_TRY(upload_bf16(m.get(), w->norm, H, &m->norm));
    {
        std::vector<const vx_qlinear_host *> p = {&w->lm_head};
        VX_TRY(upload_qlin(m.get(), p, {cfg->vocab}, H, false, &m->lm));
    }
    m->layers.resize(L);
    for (int64_t i = 0; i < L; i++) {
        const vx_layer_host &lh = w->layers[i];
        LayerDev &ld = m->layers[i];
        VX_TRY(upload_bf16(m.get(), lh.ln1, H, &ld.ln1));
        VX_TRY(upload_bf16(m.get(), lh.ln2, H, &ld.ln2));
        VX_TRY(upload_bf16(m.get(), lh.q_norm, D, &ld.qn));
        VX_TRY(upload_bf16(m.get(), lh.k_norm, D, &ld.kn));
        VX_TRY(upload_qlin(m.get(), {&lh.q, &lh.k, &lh.v}, {HQ * D, HK * D, HK * D}, H, false, &ld.qkv));
        VX_TRY(upload_qlin(m.get(), {&lh.o}, {H}, HQ * D, false, &ld.o));
        VX_TRY(upload_qlin(m.get(), {&lh.gate, &lh.up}, {F, F}, H, true, &ld.gu));
        VX_TRY(upload_qlin(m.get(), {&lh.down}, {H}, F, false, &ld.down));
    }
    // RoPE tables (qwen3.rs:278-295): f64 inv_freq -> f32, t * inv_freq in f32,
    // sin/cos in f32, then the model dtype.
    const int64_t half = D / 2;
    std::vector<float> inv(half);
    for (int64_t j = 0; j < half; j++) inv[j] = 1.0f / (float)std::pow(cfg->rope_theta, (double)(2 * j) / (double)D);
    std::vector<uint16_t> ct((size_t)(cfg->max_pos * half)), stt((size_t)(cfg->max_pos * half));
    for (int64_t t = 0; t < cfg->max_pos; t++)
        for (int64_t j = 0; j < half; j++) {
            const float f = (float)t * inv[j];
            ct[t * half + j] = f2bf(cosf(f));
            stt[t * half + j] = f2bf(sinf(f));
        }
    VX_TRY(dev_upload(m.get(), ct.data(), ct.size() * 2, (void **)&m->cos_t));
    VX_TRY(dev_upload(m.get(), stt.data(), stt.size() * 2, (void **)&m->sin_t));
    *out = m.release();
    return 0;
}

extern "C" void vx_model_destroy(vx_model *m) { delete m; }

namespace {

struct SeqDesc {
    int64_t new_tokens, kv_offset;
    const uint32_t *bt;
    int64_t n_blocks;
};

// Build the metadata blob for one forward (host side).  Fails like the
// reference when a block table is too short (qwen3.rs:682-689).
int build_meta(const vx_model *m, const vx_pages *pg, const SeqDesc *seqs, int64_t n, const int32_t *parents,
               std::vector<uint8_t> &blob, Meta &meta) {
    meta = Meta{};
    meta.n_seqs = n;
    int64_t rows = 0;
    for (int64_t s = 0; s < n; s++) {
        rows += seqs[s].new_tokens;
        meta.max_blocks = std::max(meta.max_blocks, seqs[s].n_blocks);
        meta.max_rows = std::max(meta.max_rows, seqs[s].new_tokens);
        meta.max_kv = std::max(meta.max_kv, seqs[s].kv_offset + seqs[s].new_tokens);
        if (parents && seqs[s].new_tokens != seqs[0].new_tokens)
            return set_error("forward: tree verify needs equal node counts");
    }
    meta.rows = rows;
    meta.tree = parents != nullptr;
    meta.one_row = n > 0 && rows == n && meta.max_rows == 1;
    const int64_t R = n ? seqs[0].new_tokens : 0;
    if (parents && R > 64) return set_error("forward: tree larger than 64 nodes");
    uint64_t tmask[64] = {0};
    int32_t depth[64] = {0};
    if (parents)
        for (int64_t i = 0; i < R; i++) {
            uint64_t mk = 1ull << i;
            int32_t d = 0;
            for (int32_t p = parents[i]; p >= 0; p = parents[p]) {
                mk |= 1ull << p;
                d++;
            }
            tmask[i] = mk;
            depth[i] = d;
        }
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    size_t o = 0;
    meta.o_pos = o;
    o = al(o + rows * 4);
    meta.o_page = o;
    o = al(o + rows * 4);
    meta.o_slot = o;
    o = al(o + rows * 4);
    meta.o_cu = o;
    o = al(o + (n + 1) * 4);
    meta.o_kvo = o;
    o = al(o + n * 4);
    meta.o_bt = o;
    o = al(o + n * meta.max_blocks * 4);
    meta.o_mask = o;
    o = al(o + (parents ? rows * 8 : 8));
    meta.o_last = o;
    o = al(o + n * 4);
    meta.size = o;
    blob.assign(o, 0);
    uint32_t *pos = (uint32_t *)&blob[meta.o_pos];
    uint32_t *page = (uint32_t *)&blob[meta.o_page];
    uint32_t *slot = (uint32_t *)&blob[meta.o_slot];
    uint32_t *cu = (uint32_t *)&blob[meta.o_cu];
    uint32_t *kvo = (uint32_t *)&blob[meta.o_kvo];
    uint32_t *bt = (uint32_t *)&blob[meta.o_bt];
    uint64_t *mask = (uint64_t *)&blob[meta.o_mask];
    uint32_t *last = (uint32_t *)&blob[meta.o_last];
    const int64_t ps = pg->page_size;
    int64_t row = 0;
    cu[0] = 0;
    for (int64_t s = 0; s < n; s++) {
        const SeqDesc &sd = seqs[s];
        for (int64_t b = 0; b < sd.n_blocks; b++) {
            if ((int64_t)sd.bt[b] >= pg->num_pages) return set_error("forward: block table holds an invalid page id");
            bt[s * meta.max_blocks + b] = sd.bt[b];
        }
        for (int64_t t = 0; t < sd.new_tokens; t++, row++) {
            const int64_t p = sd.kv_offset + t;
            const int64_t blk = p / ps;
            if (blk >= sd.n_blocks) return set_error("fused prefill: block_table too short");
            page[row] = sd.bt[blk];
            slot[row] = (uint32_t)(p % ps);
            const int64_t rp = sd.kv_offset + (parents ? depth[t] : t);
            if (rp >= m->cfg.max_pos) return set_error("forward: position exceeds max_position_embeddings");
            pos[row] = (uint32_t)rp;
            if (parents) mask[row] = tmask[t];
        }
        cu[s + 1] = (uint32_t)row;
        kvo[s] = (uint32_t)sd.kv_offset;
        last[s] = (uint32_t)(row - 1);
    }
    return 0;
}

int ensure_buffers(vx_model *m, int64_t rows) {
    if (rows <= m->cap_rows) return 0;
    const vx_qwen3_config &c = m->cfg;
    const int64_t H = c.hidden, F = c.inter, QW = c.n_heads * c.head_dim, KW = c.n_kv_heads * c.head_dim;
    const int64_t R = std::max<int64_t>(rows, 16);
    VX_TRY(m->h.ensure(R * H * 2));
    VX_TRY(m->xn.ensure(R * std::max({H, QW, F}) * 2));
    VX_TRY(m->q.ensure(R * QW * 2));
    VX_TRY(m->attn.ensure(R * QW * 2));
    VX_TRY(m->act.ensure(R * F * 2));
    VX_TRY(m->ids.ensure(R * 4));
    m->cap_rows = R;
    return 0;
}

// The attention launch of a layer may read the qkv projection's split
// partials (fused finish) while it writes its own split partials: its
// workspace starts past them.
size_t attn_ws_offset(int64_t rows, int64_t N, int64_t K) {
    return (qmm_partial_ws_bytes(rows, N, K) + 255) & ~(size_t)255;
}

size_t forward_ws_bytes(const vx_model *m, int64_t rows, int64_t logit_rows, int64_t n_seqs, int64_t max_rows,
                        int64_t max_kv) {
    const vx_qwen3_config &c = m->cfg;
    const int64_t H = c.hidden, F = c.inter, QW = c.n_heads * c.head_dim, KW = c.n_kv_heads * c.head_dim;
    size_t need = 0;
    need = std::max(need, qmm_partial_ws_bytes(rows, QW + 2 * KW, H));
    need = std::max(need, qmm_partial_ws_bytes(rows, H, QW));
    need = std::max(need, qmm_workspace_bytes(rows, 2 * F, H, VX_EPI_SWIGLU, true));
    need = std::max(need, qmm_partial_ws_bytes(rows, H, F));
    need = std::max(need, qmm_workspace_bytes(logit_rows, c.vocab, H, VX_EPI_STORE, true));
    // attention: upper bound on its split plan (see paged_attention_launch)
    need = std::max(need, attn_ws_offset(rows, QW + 2 * KW, H) +
                              attn_workspace_bound(n_seqs, c.n_kv_heads, max_rows, c.n_heads / c.n_kv_heads,
                                                   c.head_dim, max_kv));
    return need;
}

// Forward over `rows` rows whose token ids are already on the device.
// With amax_v set, the LM head also writes greedy-argmax partials of its
// logits ([rows, vocab / 128]) and *amax_done reports whether it did.
int forward_dev(vx_model *m, vx_pages *pg, const uint32_t *ids_dev, const Meta &meta, const uint8_t *meta_dev,
                int all_rows, void *logits, void *ws, size_t ws_bytes, hipStream_t st, Prof *prof = nullptr,
                double kv_bytes_per_layer = 0.0, float *amax_v = nullptr, uint32_t *amax_i = nullptr,
                bool *amax_done = nullptr, int64_t ids_stride = 1) {
    if (amax_done) *amax_done = false;
    const vx_qwen3_config &c = m->cfg;
    const int64_t H = c.hidden, F = c.inter, D = c.head_dim, HQ = c.n_heads, HK = c.n_kv_heads;
    const int64_t QW = HQ * D, KW = HK * D, R = meta.rows;
    const float eps = (float)c.rms_eps;
    VX_REQUIRE(pg->kv_heads == HK && pg->head_dim == D, "forward: pages do not match the model");
    VX_REQUIRE(pg->layers >= m->L, "forward: pages have fewer layers than the model");
    VX_REQUIRE(pg->dtype == VX_F16, "forward: the fused verify path keeps KV pages in f16");
    const uint32_t *pos = (const uint32_t *)(meta_dev + meta.o_pos);
    const uint32_t *pages = (const uint32_t *)(meta_dev + meta.o_page);
    const uint32_t *slots = (const uint32_t *)(meta_dev + meta.o_slot);
    const uint32_t *cu = (const uint32_t *)(meta_dev + meta.o_cu);
    const uint32_t *kvo = (const uint32_t *)(meta_dev + meta.o_kvo);
    const uint32_t *bt = (const uint32_t *)(meta_dev + meta.o_bt);
    const uint64_t *mask = meta.tree ? (const uint64_t *)(meta_dev + meta.o_mask) : nullptr;
    const uint32_t *last = (const uint32_t *)(meta_dev + meta.o_last);
    uint16_t *h = (uint16_t *)m->h.p, *xn = (uint16_t *)m->xn.p;
    uint16_t *q = (uint16_t *)m->q.p, *attn = (uint16_t *)m->attn.p, *act = (uint16_t *)m->act.p;
    const float scale = 1.0f / sqrtf((float)D);

    // Per layer: qkv projection (split partials) -> q/k norm + RoPE + KV write
    // (finishing the projection) -> attention -> o projection (partials) ->
    // residual + ln2 norm -> gate|up with the SwiGLU finish -> down
    // projection (partials) -> residual + the next norm (next layer's ln1,
    // or the final norm when every row goes to the LM head).
    {
        ProfScope ps_(prof, st, PC_OTHER, 0.0);
        VX_TRY(embed_rmsnorm_launch(ids_dev, ids_stride, m->embed, c.vocab, m->layers[0].ln1, h, xn, R, H, eps,
                                    VX_F16, st));
    }
    int splits = 0;
    const float *part = nullptr;
    // Opt-in (VX_FUSED_QKV=1): with one query tile per sequence (up to 64
    // query vectors for head_dim <= 128, 32 above) attention can finish
    // q/k/v itself.  It is bit-identical to the separate kernel but measured
    // slower at the bench shape (27.7 us against 5.4 + 11.0 us): the
    // finish adds four dependent memory round trips ahead of the key loop on
    // 128 workgroups, where the separate kernel spreads them over the chip.
    // The final norm runs inside the last layer's residual kernel when every
    // row goes to the LM head: all rows, or one row per sequence (a draft
    // step, where row s is sequence s's last row); otherwise a gather of the
    // last rows follows the layers.
    const bool norm_all = all_rows || meta.one_row;
    const int64_t G = HQ / HK;
    const char *fz_env = getenv("VX_FUSED_QKV");
    const bool fuse_qkv = meta.max_rows * G <= (D <= 128 ? 64 : 32) && fz_env && atoi(fz_env) != 0;
    for (int64_t l = 0; l < m->L; l++) {
        const LayerDev &ly = m->layers[l];
        uint16_t *kp = (uint16_t *)vx_pages_pool(pg, l, 0);
        uint16_t *vp = (uint16_t *)vx_pages_pool(pg, l, 1);
        {
            ProfScope ps_(prof, st, PC_QMM, qmm_bytes(R, QW + 2 * KW, H, false));
            VX_TRY(qmm_packed_partial(xn, ly.qkv.packed, R, QW + 2 * KW, H, ws, ws_bytes, &splits, &part, st));
        }
        if (fuse_qkv) {
            // q/k norm, RoPE and the KV write happen inside the attention launch
            const AttnQkvFuse fz{part, splits, ly.qn, ly.kn, m->cos_t, m->sin_t, pos, pages, slots, eps};
            const size_t off = attn_ws_offset(R, QW + 2 * KW, H);
            ProfScope ps_(prof, st, PC_ATTN, kv_bytes_per_layer + 4.0 * R * QW);
            VX_TRY(paged_attention_launch(nullptr, kp, vp, bt, cu, kvo, mask, attn, 0, R, meta.n_seqs,
                                          meta.max_rows, meta.max_blocks, pg->num_pages, HQ, HK, D, pg->page_size,
                                          scale, 0, VX_F16, (char *)ws + off, ws_bytes - off, meta.max_kv, st, 1,
                                          &fz));
        } else {
            {
                ProfScope ps_(prof, st, PC_OTHER, 0.0);
                VX_TRY(qkv_partial_rope_scatter_launch(part, splits, ly.qn, ly.kn, m->cos_t, m->sin_t, pos, pages,
                                                       slots, q, kp, vp, R, (int)HQ, (int)HK, (int)D,
                                                       (int)pg->page_size, eps, VX_F16, st));
            }
            ProfScope ps_(prof, st, PC_ATTN, kv_bytes_per_layer + 4.0 * R * QW);
            VX_TRY(paged_attention_launch(q, kp, vp, bt, cu, kvo, mask, attn, 0, R, meta.n_seqs, meta.max_rows,
                                          meta.max_blocks, pg->num_pages, HQ, HK, D, pg->page_size, scale, 0,
                                          VX_F16, ws, ws_bytes, meta.max_kv, st, 1, nullptr));
        }
        {
            ProfScope ps_(prof, st, PC_QMM, qmm_bytes(R, H, QW, true));
            VX_TRY(qmm_packed_partial(attn, ly.o.packed, R, H, QW, ws, ws_bytes, &splits, &part, st));
        }
        {
            ProfScope ps_(prof, st, PC_OTHER, 0.0);
            VX_TRY(residual_rmsnorm_launch(part, splits, 1.0f, h, ly.ln2, xn, R, H, eps, VX_F16, st));
        }
        {
            ProfScope ps_(prof, st, PC_QMM, qmm_bytes(R, 2 * F, H, false) - 2.0 * R * F);
            VX_TRY(qmm_packed(xn, ly.gu.packed, act, nullptr, R, 2 * F, H, 0, kMlpShift, VX_BF16,
                              VX_F16, VX_EPI_SWIGLU, ws, ws_bytes, st));
        }
        {
            ProfScope ps_(prof, st, PC_QMM, qmm_bytes(R, H, F, true));
            VX_TRY(qmm_packed_partial(act, ly.down.packed, R, H, F, ws, ws_bytes, &splits, &part, st));
        }
        {
            ProfScope ps_(prof, st, PC_OTHER, 0.0);
            const bool last_layer = l + 1 == m->L;
            const uint16_t *next_ln = !last_layer ? m->layers[l + 1].ln1 : (norm_all ? m->norm : nullptr);
            VX_TRY(residual_rmsnorm_launch(part, splits, ldexpf(1.0f, kMlpShift), h, next_ln, xn, R, H, eps,
                                           VX_F16, st));
        }
    }
    const int64_t lrows = all_rows ? R : meta.n_seqs;
    if (!norm_all) {
        ProfScope ps_(prof, st, PC_OTHER, 0.0);
        VX_TRY(rmsnorm_launch(h, m->norm, xn, last, lrows, H, eps, VX_F16, st));
    }
    {
        ProfScope ps_(prof, st, PC_QMM, qmm_bytes(lrows, c.vocab, H, false));
        if (amax_v && qmm_packed_argmax_ok(lrows, c.vocab, H)) {
            VX_TRY(qmm_packed_argmax(xn, m->lm.packed, logits, lrows, c.vocab, H, VX_BF16, VX_BF16, amax_v, amax_i,
                                     ws, ws_bytes, st));
            if (amax_done) *amax_done = true;
        } else {
            VX_TRY(qmm_packed(xn, m->lm.packed, logits, nullptr, lrows, c.vocab, H, 0, 0, VX_BF16, VX_BF16,
                              VX_EPI_STORE, ws, ws_bytes, st));
        }
    }
    return 0;
}

int prepare_ws(vx_model *m, const Meta &meta, int all_rows) {
    const size_t need = forward_ws_bytes(m, meta.rows, all_rows ? meta.rows : meta.n_seqs, meta.n_seqs,
                                         meta.max_rows, meta.max_kv);
    if (m->ws.n < need) {
        VX_HIP(hipDeviceSynchronize());
        VX_TRY(m->ws.ensure(need));
        VX_HIP(hipMemset(m->ws.p, 0, m->ws.n));
    }
    return 0;
}

}  // namespace

extern "C" int vx_forward(vx_model *m, vx_pages *pages, const uint32_t *input_ids, const vx_seq_slice *seqs,
                          int64_t n_seqs, int all_rows, const int32_t *tree_parents, void *logits,
                          void *stream) {
    // the tree is checked before anything reads it (its ancestor walk
    // assumes parents[j] < j)
    if (tree_parents && seqs && n_seqs > 0) VX_TRY(check_tree_parents(tree_parents, seqs[0].new_tokens, "forward"));
    VX_REQUIRE(m && pages && input_ids && seqs && logits, "forward: null argument");
    hipStream_t st = (hipStream_t)stream;
    std::vector<SeqDesc> sd(n_seqs);
    for (int64_t i = 0; i < n_seqs; i++) sd[i] = {seqs[i].new_tokens, seqs[i].kv_offset, seqs[i].block_table, seqs[i].n_blocks};
    std::vector<uint8_t> blob;
    Meta meta;
    VX_TRY(build_meta(m, pages, sd.data(), n_seqs, tree_parents, blob, meta));
    if (meta.rows == 0) return 0;
    for (int64_t i = 0; i < meta.rows; i++)
        VX_REQUIRE(input_ids[i] < (uint32_t)m->cfg.vocab, "forward: token id out of range");
    VX_TRY(ensure_buffers(m, meta.rows));
    VX_TRY(m->meta.ensure(meta.size));
    VX_TRY(prepare_ws(m, meta, all_rows));
    VX_HIP(hipMemcpyAsync(m->meta.p, blob.data(), meta.size, hipMemcpyHostToDevice, st));
    VX_HIP(hipMemcpyAsync(m->ids.p, input_ids, meta.rows * 4, hipMemcpyHostToDevice, st));
    VX_TRY(forward_dev(m, pages, (const uint32_t *)m->ids.p, meta, (const uint8_t *)m->meta.p, all_rows, logits,
                       m->ws.p, m->ws.n, st));
    // the host blob must outlive the async copy
    VX_HIP(hipStreamSynchronize(st));
    return 0;
}

// ===========================================================================
// spec engine (spec.rs)
// ===========================================================================
namespace {
struct SpecState {
    std::vector<uint32_t> target_blocks, draft_blocks;
    int64_t kv_len = 0;
    uint32_t last_token = 0;
    std::vector<uint32_t> tokens;
    uint32_t stream_id = 0, round = 0;
    float temperature = 0.f;
    int64_t prompt_len = 0;  // tokens[0, prompt_len) is the prompt
    bool live = false;
    bool ready = false;      // prompt[..len-1] is in both caches: rounds may run
};
}  // namespace

struct vx_spec {
    vx_model *target, *draft;
    vx_pages *tp, *dp;
    float temperature;
    uint64_t seed;
    int fix_hole;
    std::vector<SpecState> states;
    // device buffers for a round
    DevBuf d_res, d_vids, d_tlog, d_dlog, d_uni, d_meta, d_argws, d_draw;  // d_res: accepted | tokens | candidates
    DevBuf d_amax;  // greedy-argmax partials written by the LM heads: values then indices
    DevBuf d_plog;  // prefill-chunk logits (discarded, spec.rs:172-173)
    // host staging (pinned)
    void *h_stage = nullptr;
    size_t h_stage_n = 0;
    std::vector<uint32_t> last_cand;
    std::vector<float> last_logits;
    int64_t last_n = 0, last_k = 0;
    // round trace: with tracing on, every draft step keeps its logits
    bool tracing = false;
    bool last_kept_draft = false;
    float last_temp = 0.f;
    uint64_t serial = 0;
    std::vector<int64_t> last_ids;
    std::vector<uint32_t> last_streams, last_rounds;
    Prof prof_draft, prof_verify;
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    int profiling = 0;
    vx_step_profile last_prof{};
    ~vx_spec() {
        if (h_stage) (void)hipHostFree(h_stage);
        for (hipEvent_t x : ev)
            if (x) (void)hipEventDestroy(x);
    }
};

extern "C" int vx_spec_create(vx_model *target, vx_pages *target_pages, vx_model *draft, vx_pages *draft_pages,
                              float temperature, uint64_t sample_seed, int fix_draft_hole, vx_spec **out) {
    VX_REQUIRE(target && target_pages && draft && draft_pages && out, "spec: null argument");
    if (target->cfg.vocab != draft->cfg.vocab)
        return set_error("draft vocab_size (" + std::to_string(draft->cfg.vocab) + ") != target vocab_size (" +
                         std::to_string(target->cfg.vocab) + "); spec decoding requires matched tokenizers");
    auto e = std::make_unique<vx_spec>();
    e->target = target;
    e->draft = draft;
    e->tp = target_pages;
    e->dp = draft_pages;
    e->temperature = temperature;
    e->seed = sample_seed;
    e->fix_hole = fix_draft_hole;
    *out = e.release();
    return 0;
}

extern "C" void vx_spec_destroy(vx_spec *e) { delete e; }
extern "C" void vx_spec_free(vx_spec *e, int64_t s);

namespace {
int page_size_or_err(const vx_spec *e, int64_t *ps) {
    if (e->dp->page_size != e->tp->page_size)
        return set_error("draft page_size (" + std::to_string(e->dp->page_size) + ") != target page_size (" +
                         std::to_string(e->tp->page_size) + ")");
    *ps = e->tp->page_size;
    return 0;
}

int ensure_capacity(vx_pages *p, std::vector<uint32_t> &bt, int64_t needed, const char *ctx) {
    if ((int64_t)bt.size() >= needed) return 0;
    std::vector<uint32_t> extra(needed - bt.size());
    if (vx_pages_alloc(p, (int64_t)extra.size(), extra.data()) != 0)
        return set_error(std::string(ctx) + ": alloc extra pages");
    bt.insert(bt.end(), extra.begin(), extra.end());
    return 0;
}

int stage(vx_spec *e, size_t bytes) {
    if (e->h_stage_n >= bytes) return 0;
    if (e->h_stage) VX_HIP(hipHostFree(e->h_stage));
    e->h_stage = nullptr;
    VX_HIP(hipHostMalloc(&e->h_stage, bytes, hipHostMallocDefault));
    e->h_stage_n = bytes;
    return 0;
}
}  // namespace

extern "C" int vx_spec_prefill(vx_spec *e, const uint32_t *const *prompts, const int64_t *lens, int64_t n,
                               int64_t *out_first_state) {
    VX_REQUIRE(e && prompts && lens && out_first_state, "prefill: null argument");
    int64_t ps;
    VX_TRY(page_size_or_err(e, &ps));
    for (int64_t b = 0; b < n; b++)
        VX_REQUIRE(lens[b] >= 2, "speculative prefill requires a prompt with at least 2 tokens");
    const int64_t first = (int64_t)e->states.size();
    std::vector<SeqDesc> ts(n), ds(n);
    std::vector<uint32_t> ids;
    auto rollback = [&]() {
        while ((int64_t)e->states.size() > first) {
            vx_spec_free(e, (int64_t)e->states.size() - 1);
            e->states.pop_back();
        }
        return -1;
    };
    for (int64_t b = 0; b < n; b++) {
        SpecState s;
        const int64_t head = lens[b] - 1;
        const int64_t need = (head + 1 + ps - 1) / ps;
        s.stream_id = (uint32_t)(first + b);
        if (ensure_capacity(e->tp, s.target_blocks, need, "alloc target prefill pages")) return rollback();
        if (ensure_capacity(e->dp, s.draft_blocks, need, "alloc draft prefill pages")) {
            vx_pages_free(e->tp, s.target_blocks.data(), (int64_t)s.target_blocks.size());
            return rollback();
        }
        s.kv_len = head;
        s.last_token = prompts[b][head];
        s.tokens.assign(prompts[b], prompts[b] + lens[b]);
        s.prompt_len = lens[b];
        s.temperature = e->temperature;
        s.live = true;
        s.ready = true;
        e->states.push_back(std::move(s));
        ids.insert(ids.end(), prompts[b], prompts[b] + head);
    }
    for (int64_t b = 0; b < n; b++) {
        SpecState &s = e->states[first + b];
        ts[b] = {lens[b] - 1, 0, s.target_blocks.data(), (int64_t)s.target_blocks.size()};
        ds[b] = {lens[b] - 1, 0, s.draft_blocks.data(), (int64_t)s.draft_blocks.size()};
    }
    // prefill both models on prompt[..len-1]; logits discarded (spec.rs:172-173)
    DevBuf lg;
    VX_TRY(lg.ensure((size_t)n * e->target->cfg.vocab * 2));
    std::vector<vx_seq_slice> sl(n);
    for (int64_t b = 0; b < n; b++) sl[b] = {ts[b].new_tokens, 0, ts[b].bt, ts[b].n_blocks};
    if (vx_forward(e->target, e->tp, ids.data(), sl.data(), n, 0, nullptr, lg.p, nullptr)) return rollback();
    for (int64_t b = 0; b < n; b++) sl[b] = {ds[b].new_tokens, 0, ds[b].bt, ds[b].n_blocks};
    if (vx_forward(e->draft, e->dp, ids.data(), sl.data(), n, 0, nullptr, lg.p, nullptr)) return rollback();
    *out_first_state = first;
    return 0;
}

extern "C" int vx_spec_add_state(vx_spec *e, const uint32_t *prompt, int64_t len, int64_t cached_tokens,
                                 const uint32_t *target_pages, const uint32_t *draft_pages, int64_t reserve_tokens,
                                 uint32_t stream_id, float temperature, int64_t *out_state) {
    VX_REQUIRE(e && prompt && out_state, "add_state: null argument");
    int64_t ps;
    VX_TRY(page_size_or_err(e, &ps));
    VX_REQUIRE(len >= 2, "speculative prefill requires a prompt with at least 2 tokens");
    VX_REQUIRE(cached_tokens >= 0 && cached_tokens <= len - 1 && cached_tokens % ps == 0,
               "add_state: cached_tokens must be a multiple of page_size and at most len - 1");
    VX_REQUIRE(cached_tokens == 0 || (target_pages && draft_pages), "add_state: cached pages missing");
    SpecState s;
    const int64_t nc = cached_tokens / ps;
    s.target_blocks.assign(target_pages, target_pages + nc);
    s.draft_blocks.assign(draft_pages, draft_pages + nc);
    const int64_t need = (std::max(reserve_tokens, len - 1) + ps - 1) / ps;
    // all-or-nothing over both pools: the caller's cached references stay its own on failure
    if (need - nc > vx_pages_num_free(e->tp) || need - nc > vx_pages_num_free(e->dp))
        return set_error("add_state: not enough free pages");
    {
        std::vector<uint32_t> t = s.target_blocks, d = s.draft_blocks;
        VX_TRY(ensure_capacity(e->tp, t, need, "alloc target pages"));
        if (ensure_capacity(e->dp, d, need, "alloc draft pages")) {
            vx_pages_free(e->tp, t.data() + nc, (int64_t)t.size() - nc);
            return -1;
        }
        s.target_blocks.swap(t);
        s.draft_blocks.swap(d);
    }
    s.kv_len = cached_tokens;
    s.tokens.assign(prompt, prompt + len);
    s.prompt_len = len;
    s.stream_id = stream_id;
    s.temperature = temperature < 0.f ? e->temperature : temperature;
    s.live = true;
    s.ready = cached_tokens == len - 1;
    if (s.ready) s.last_token = prompt[len - 1];
    int64_t slot = 0;
    while (slot < (int64_t)e->states.size() && e->states[slot].live) slot++;
    if (slot == (int64_t)e->states.size()) e->states.emplace_back();
    e->states[slot] = std::move(s);
    *out_state = slot;
    return 0;
}

extern "C" int vx_spec_prefill_chunk(vx_spec *e, const int64_t *state_ids, const int64_t *n_tokens, int64_t n,
                                     void *stream) {
    VX_REQUIRE(e && (n == 0 || (state_ids && n_tokens)), "prefill_chunk: null argument");
    int64_t ps;
    VX_TRY(page_size_or_err(e, &ps));
    if (n == 0) return 0;
    std::vector<SpecState *> S(n);
    std::vector<uint32_t> ids;
    for (int64_t b = 0; b < n; b++) {
        VX_REQUIRE(state_ids[b] >= 0 && state_ids[b] < (int64_t)e->states.size() && e->states[state_ids[b]].live,
                   "prefill_chunk: unknown state");
        SpecState &s = e->states[state_ids[b]];
        VX_REQUIRE(!s.ready, "prefill_chunk: state has no prompt left to prefill");
        VX_REQUIRE(n_tokens[b] >= 1 && s.kv_len + n_tokens[b] <= s.prompt_len - 1,
                   "prefill_chunk: chunk runs past prompt[..len-1]");
        for (int64_t c = 0; c < b; c++)
            VX_REQUIRE(state_ids[c] != state_ids[b], "prefill_chunk: state listed twice");
        S[b] = &s;
    }
    for (int64_t b = 0; b < n; b++) {
        const int64_t end = S[b]->kv_len + n_tokens[b];
        VX_TRY(ensure_capacity(e->tp, S[b]->target_blocks, (end + ps - 1) / ps, "alloc target prefill pages"));
        VX_TRY(ensure_capacity(e->dp, S[b]->draft_blocks, (end + ps - 1) / ps, "alloc draft prefill pages"));
        ids.insert(ids.end(), S[b]->tokens.begin() + S[b]->kv_len, S[b]->tokens.begin() + end);
    }
    VX_TRY(e->d_plog.ensure((size_t)n * e->target->cfg.vocab * 2));
    std::vector<vx_seq_slice> sl(n);
    for (int64_t b = 0; b < n; b++)
        sl[b] = {n_tokens[b], S[b]->kv_len, S[b]->target_blocks.data(), (int64_t)S[b]->target_blocks.size()};
    VX_TRY(vx_forward(e->target, e->tp, ids.data(), sl.data(), n, 0, nullptr, e->d_plog.p, stream));
    for (int64_t b = 0; b < n; b++)
        sl[b] = {n_tokens[b], S[b]->kv_len, S[b]->draft_blocks.data(), (int64_t)S[b]->draft_blocks.size()};
    VX_TRY(vx_forward(e->draft, e->dp, ids.data(), sl.data(), n, 0, nullptr, e->d_plog.p, stream));
    for (int64_t b = 0; b < n; b++) {
        SpecState &s = *S[b];
        s.kv_len += n_tokens[b];
        if (s.kv_len == s.prompt_len - 1) {
            s.ready = true;
            s.last_token = s.tokens[s.prompt_len - 1];
        }
    }
    return 0;
}

extern "C" int64_t vx_spec_state_pages(const vx_spec *e, int64_t s, int which, uint32_t *out, int64_t cap) {
    if (!e || s < 0 || s >= (int64_t)e->states.size() || !e->states[s].live) return -1;
    const auto &bt = which ? e->states[s].draft_blocks : e->states[s].target_blocks;
    if (out) memcpy(out, bt.data(), (size_t)std::min<int64_t>(cap, (int64_t)bt.size()) * 4);
    return (int64_t)bt.size();
}

namespace {
__global__ void build_verify_ids(const uint32_t *last, const uint32_t *cand, uint32_t *vids, int64_t n, int64_t k) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * (k + 1)) return;
    const int64_t b = i / (k + 1), j = i % (k + 1);
    vids[i] = j == 0 ? last[b] : cand[b * k + j - 1];
}
__global__ void spec_uniforms_kernel(float *out, const uint32_t *streams, const uint32_t *rounds, int64_t n,
                                     int64_t k, uint32_t k0, uint32_t k1) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * (k + 1)) return;
    const int64_t b = i / (k + 1), j = i % (k + 1);
    uint32_t c[4] = {streams[b], rounds[b], (uint32_t)j, 0u};
    vx_philox(c, k0, k1);
    for (int t = 0; t < 4; t++) out[i * 4 + t] = vx_u01(c[t]);
}
}  // namespace

extern "C" int vx_spec_step(vx_spec *e, const int64_t *state_ids, int64_t n, int64_t draft_k, int64_t eos,
                            vx_round_outcome *outcomes, uint32_t *committed, void *stream) {
    VX_REQUIRE(e && state_ids && outcomes && committed, "step: null argument");
    if (draft_k == 0) return set_error("draft_k must be >= 1");
    VX_REQUIRE(draft_k > 0 && draft_k + 1 <= 64, "step: draft_k out of range");
    int64_t ps;
    VX_TRY(page_size_or_err(e, &ps));
    hipStream_t st = (hipStream_t)stream;
    const int64_t D = draft_k, V = e->target->cfg.vocab;
    std::vector<SpecState *> S(n);
    for (int64_t b = 0; b < n; b++) {
        VX_REQUIRE(state_ids[b] >= 0 && state_ids[b] < (int64_t)e->states.size() && e->states[state_ids[b]].live,
                   "step: unknown state");
        S[b] = &e->states[state_ids[b]];
        VX_REQUIRE(S[b]->ready, "step: state is still prefilling");
        VX_REQUIRE(S[b]->temperature == S[0]->temperature, "step: states of one round must share a temperature");
    }
    const float temp = n > 0 ? S[0]->temperature : e->temperature;
    // capacity (spec.rs:198-205)
    for (int64_t b = 0; b < n; b++) {
        VX_TRY(ensure_capacity(e->tp, S[b]->target_blocks, (S[b]->kv_len + D + 1 + ps - 1) / ps, "grow target block table"));
        VX_TRY(ensure_capacity(e->dp, S[b]->draft_blocks, (S[b]->kv_len + D + ps - 1) / ps, "grow draft block table"));
    }
    // metadata for D draft forwards + 1 verify forward
    std::vector<std::vector<uint8_t>> blobs(D + 1);
    std::vector<Meta> metas(D + 1);
    std::vector<SeqDesc> sd(n);
    for (int64_t i = 0; i < D; i++) {
        for (int64_t b = 0; b < n; b++)
            sd[b] = {1, S[b]->kv_len + i, S[b]->draft_blocks.data(), (int64_t)S[b]->draft_blocks.size()};
        VX_TRY(build_meta(e->draft, e->dp, sd.data(), n, nullptr, blobs[i], metas[i]));
    }
    for (int64_t b = 0; b < n; b++)
        sd[b] = {D + 1, S[b]->kv_len, S[b]->target_blocks.data(), (int64_t)S[b]->target_blocks.size()};
    VX_TRY(build_meta(e->target, e->tp, sd.data(), n, nullptr, blobs[D], metas[D]));
    std::vector<size_t> boff(D + 1);
    size_t total = 0;
    for (int64_t i = 0; i <= D; i++) {
        boff[i] = total;
        total += (metas[i].size + 255) & ~(size_t)255;
    }
    const size_t small = (size_t)n * 4 * 3;  // last tokens, stream ids, rounds
    const size_t res_bytes = (size_t)n * 4 + (size_t)n * (D + 1) * 4 + (size_t)n * D * 4;
    VX_TRY(stage(e, total + small + res_bytes + 256));
    uint8_t *hs = (uint8_t *)e->h_stage;
    for (int64_t i = 0; i <= D; i++) memcpy(hs + boff[i], blobs[i].data(), metas[i].size);
    uint32_t *h_last = (uint32_t *)(hs + total);
    uint32_t *h_strm = h_last + n;
    uint32_t *h_rnd = h_strm + n;
    for (int64_t b = 0; b < n; b++) {
        h_last[b] = S[b]->last_token;
        h_strm[b] = S[b]->stream_id;
        h_rnd[b] = S[b]->round;
    }
    // device buffers
    VX_TRY(ensure_buffers(e->draft, n));
    VX_TRY(ensure_buffers(e->target, n * (D + 1)));
    VX_TRY(e->d_meta.ensure(total + small));
    VX_TRY(e->d_res.ensure(res_bytes));
    VX_TRY(e->d_vids.ensure(n * (D + 1) * 4));
    VX_TRY(e->d_tlog.ensure((size_t)n * (D + 1) * V * 2));
    const bool stoch = temp > 0.f;
    const bool keep_draft = stoch || e->tracing;  // draft logits laid out [D][n][V] (step-major)
    VX_TRY(e->d_dlog.ensure((size_t)n * (keep_draft ? D : 1) * V * 2));
    VX_TRY(e->d_uni.ensure(n * (D + 1) * 16));
    VX_TRY(e->d_draw.ensure(n * 4));
    const int64_t amax_chunks = vx_cdiv(V, 128);
    VX_TRY(e->d_amax.ensure((size_t)n * (D + 1) * amax_chunks * 8));
    float *amax_v = (float *)e->d_amax.p;
    uint32_t *amax_i = (uint32_t *)(amax_v + n * (D + 1) * amax_chunks);
    size_t accws = std::max(accept_workspace_bytes(n * (D + 1), V), stochastic_workspace_bytes(n * (2 * D + 1), V));
    if (e->d_argws.n < accws) {
        VX_HIP(hipDeviceSynchronize());
        VX_TRY(e->d_argws.ensure(accws));
        VX_HIP(hipMemset(e->d_argws.p, 0, e->d_argws.n));
    }
    VX_TRY(prepare_ws(e->draft, metas[0], 0));
    VX_TRY(prepare_ws(e->target, metas[D], 1));
    uint8_t *dm = (uint8_t *)e->d_meta.p;
    VX_HIP(hipMemcpyAsync(dm, hs, total + small, hipMemcpyHostToDevice, st));
    const uint32_t *d_last = (const uint32_t *)(dm + total);
    // the round's results in one buffer laid out like the host stage: accepted
    // lengths [n], committed tokens [n, D+1], candidates [n, D]
    int32_t *d_acc = (int32_t *)e->d_res.p;
    uint32_t *d_tok = (uint32_t *)((uint8_t *)e->d_res.p + n * 4);
    uint32_t *cand = d_tok + n * (D + 1);
    float *uni = (float *)e->d_uni.p;
    if (stoch) {
        hipLaunchKernelGGL(spec_uniforms_kernel, dim3((unsigned)vx_cdiv(n * (D + 1), 256)), dim3(256), 0, st, uni,
                           d_last + n, d_last + 2 * n, n, D, (uint32_t)e->seed, (uint32_t)(e->seed >> 32));
        VX_HIP(hipGetLastError());
    }
    // profiling 1: events around every kernel and at the phase boundaries;
    // 2: phase boundaries only (the round runs undisturbed)
    const bool prof = e->profiling != 0;
    const bool per_kernel = e->profiling == 1;
    if (prof) {
        for (int j = 0; j < 4; j++)
            if (!e->ev[j]) VX_HIP(hipEventCreate(&e->ev[j]));
        e->prof_draft.reset();
        e->prof_verify.reset();
        e->prof_draft.on = e->prof_verify.on = per_kernel;
        VX_HIP(hipEventRecord(e->ev[0], st));
    }
    // KV bytes read per verify layer (K and V of every visible position)
    double kv_verify = 0.0, kv_draft = 0.0;
    for (int64_t b = 0; b < n; b++) {
        kv_verify += (double)(S[b]->kv_len + D + 1) * e->tp->kv_heads * e->tp->head_dim * 2 * 2;
        kv_draft += (double)(S[b]->kv_len + (D + 1) / 2.0) * e->dp->kv_heads * e->dp->head_dim * 2 * 2;
    }
    // ---- draft phase: feed [last, c0 .. c_{D-2}] (spec.rs:223-240)
    for (int64_t i = 0; i < D; i++) {
        void *dl = keep_draft ? (void *)((uint16_t *)e->d_dlog.p + (size_t)i * n * V) : e->d_dlog.p;
        bool fused_amax = false;
        // step i's input: the last tokens, then column i - 1 of cand [n, D]
        const uint32_t *in_ids = i == 0 ? d_last : cand + (i - 1);
        VX_TRY(forward_dev(e->draft, e->dp, in_ids, metas[i], dm + boff[i], 0, dl, e->draft->ws.p, e->draft->ws.n,
                           st, per_kernel ? &e->prof_draft : nullptr, kv_draft, stoch ? nullptr : amax_v, amax_i,
                           &fused_amax, i == 0 ? 1 : D));
        if (!stoch && fused_amax) {
            VX_TRY(argmax_accept_partials_launch(amax_v, amax_i, (int)amax_chunks, n, 0, 1, nullptr, 0, nullptr,
                                                 nullptr, cand + i, D, st));
        } else if (!stoch) {
            VX_TRY(argmax_accept_launch(dl, VX_BF16, n, V, 0, 1, nullptr, 0, nullptr, nullptr, nullptr, nullptr,
                                        nullptr, cand + i, D, e->d_argws.p, e->d_argws.n, st));
        } else {
            VX_TRY(sample_rows_launch(dl, VX_BF16, uni + i * 4, (D + 1) * 4, (uint32_t *)e->d_draw.p, n, V,
                                      temp, cand + i, D, e->d_argws.p, e->d_argws.n, st));
        }
    }
    // ---- verify (spec.rs:246-264)
    hipLaunchKernelGGL(build_verify_ids, dim3((unsigned)vx_cdiv(n * (D + 1), 256)), dim3(256), 0, st, d_last, cand,
                       (uint32_t *)e->d_vids.p, n, D);
    VX_HIP(hipGetLastError());
    if (prof) VX_HIP(hipEventRecord(e->ev[1], st));
    bool verify_amax = false;
    VX_TRY(forward_dev(e->target, e->tp, (const uint32_t *)e->d_vids.p, metas[D], dm + boff[D], 1, e->d_tlog.p,
                       e->target->ws.p, e->target->ws.n, st, per_kernel ? &e->prof_verify : nullptr, kv_verify,
                       stoch ? nullptr : amax_v, amax_i, &verify_amax));
    if (prof) VX_HIP(hipEventRecord(e->ev[2], st));
    // ---- acceptance (spec.rs:266-292)
    if (!stoch && verify_amax) {
        VX_TRY(argmax_accept_partials_launch(amax_v, amax_i, (int)amax_chunks, n * (D + 1), 1, (int)(D + 1), cand,
                                             (int)D, d_acc, d_tok, nullptr, 0, st));
    } else if (!stoch) {
        VX_TRY(argmax_accept_launch(e->d_tlog.p, VX_BF16, n * (D + 1), V, 1, (int)(D + 1), cand, (int)D,
                                    d_acc, d_tok, nullptr, nullptr, nullptr, nullptr,
                                    0, e->d_argws.p, e->d_argws.n, st));
    } else {
        // draft logits are laid out [D][n][V] (step-major)
        VX_TRY(stochastic_accept_launch(e->d_tlog.p, e->d_dlog.p, VX_BF16, cand, uni, d_acc,
                                        d_tok, n, D, V, temp, true, e->d_argws.p, e->d_argws.n,
                                        st));
    }
    // ---- results to host (one copy set, one sync)
    uint8_t *hr = hs + total + small;
    int32_t *h_acc = (int32_t *)hr;
    uint32_t *h_tok = (uint32_t *)(hr + n * 4);
    uint32_t *h_cand = h_tok + n * (D + 1);
    VX_HIP(hipMemcpyAsync(hr, e->d_res.p, res_bytes, hipMemcpyDeviceToHost, st));
    if (prof) VX_HIP(hipEventRecord(e->ev[3], st));
    VX_HIP(hipStreamSynchronize(st));
    if (prof) {
        vx_step_profile &pp = e->last_prof;
        pp = vx_step_profile{};
        float ms = 0.f;
        VX_HIP(hipEventElapsedTime(&ms, e->ev[0], e->ev[1]));
        pp.draft_ms = ms;
        VX_HIP(hipEventElapsedTime(&ms, e->ev[1], e->ev[2]));
        pp.verify_ms = ms;
        VX_HIP(hipEventElapsedTime(&ms, e->ev[2], e->ev[3]));
        pp.accept_ms = ms;
        for (auto *pr : {&e->prof_verify, &e->prof_draft}) {
            const bool ver = pr == &e->prof_verify;
            for (const auto &r : pr->recs) {
                VX_HIP(hipEventElapsedTime(&ms, r.a, r.b));
                if (ver) {
                    pp.verify_kernel_ms[r.cls] += ms;
                    pp.verify_kernel_bytes[r.cls] += r.bytes;
                    pp.verify_kernel_launches[r.cls] += 1;
                } else {
                    pp.draft_kernel_ms[r.cls] += ms;
                    pp.draft_kernel_bytes[r.cls] += r.bytes;
                    pp.draft_kernel_launches[r.cls] += 1;
                }
            }
        }
    }
    e->last_n = n;
    e->last_k = D;
    e->last_cand.assign(h_cand, h_cand + n * D);
    e->last_kept_draft = keep_draft;
    e->last_temp = temp;
    e->serial++;
    e->last_ids.assign(state_ids, state_ids + n);
    e->last_streams.assign(h_strm, h_strm + n);
    e->last_rounds.assign(h_rnd, h_rnd + n);
    // ---- commit (spec.rs:294-309)
    for (int64_t b = 0; b < n; b++) {
        SpecState &s = *S[b];
        const int32_t a = h_acc[b];
        VX_REQUIRE(a >= 0 && a <= D, "step: acceptance returned an invalid count");
        for (int32_t i = 0; i <= a; i++) committed[b * (D + 1) + i] = h_tok[b * (D + 1) + i];
        if (e->fix_hole && a == D) {
            // opt-in: feed c[D-1] to the draft so its KV has no unwritten slot
            VX_TRY(ensure_capacity(e->dp, s.draft_blocks, (s.kv_len + D + 1 + ps - 1) / ps, "grow draft block table"));
            vx_seq_slice one = {1, s.kv_len + D, s.draft_blocks.data(), (int64_t)s.draft_blocks.size()};
            DevBuf lg;
            VX_TRY(lg.ensure((size_t)V * 2));
            const uint32_t id = h_cand[b * D + D - 1];
            VX_TRY(vx_forward(e->draft, e->dp, &id, &one, 1, 0, nullptr, lg.p, stream));
        }
        s.kv_len += a + 1;
        s.last_token = h_tok[b * (D + 1) + a];
        s.tokens.insert(s.tokens.end(), h_tok + b * (D + 1), h_tok + b * (D + 1) + a + 1);
        s.round++;
        int stop = 0;
        if (eos >= 0)
            for (int32_t i = 0; i <= a; i++)
                if (h_tok[b * (D + 1) + i] == (uint32_t)eos) stop = 1;
        outcomes[b] = {a, a + 1, stop};
    }
    return 0;
}

extern "C" int64_t vx_spec_state_kv_len(const vx_spec *e, int64_t s) {
    if (!e || s < 0 || s >= (int64_t)e->states.size()) return -1;
    return e->states[s].kv_len;
}
extern "C" int64_t vx_spec_state_num_tokens(const vx_spec *e, int64_t s) {
    if (!e || s < 0 || s >= (int64_t)e->states.size()) return -1;
    return (int64_t)e->states[s].tokens.size();
}
extern "C" int vx_spec_state_tokens(const vx_spec *e, int64_t s, uint32_t *out, int64_t cap) {
    VX_REQUIRE(e && s >= 0 && s < (int64_t)e->states.size() && out, "state: bad argument");
    const auto &t = e->states[s].tokens;
    VX_REQUIRE(cap >= (int64_t)t.size(), "state: output too small");
    memcpy(out, t.data(), t.size() * 4);
    return 0;
}
extern "C" int vx_spec_last_trace(const vx_spec *e, uint32_t *candidates, float *verify_logits) {
    VX_REQUIRE(e && e->last_n > 0, "trace: no step yet");
    if (candidates) memcpy(candidates, e->last_cand.data(), e->last_cand.size() * 4);
    if (verify_logits) {
        const int64_t n = e->last_n * (e->last_k + 1) * e->target->cfg.vocab;
        std::vector<uint16_t> tmp((size_t)n);
        VX_HIP(hipMemcpy(tmp.data(), e->d_tlog.p, (size_t)n * 2, hipMemcpyDeviceToHost));
        for (int64_t i = 0; i < n; i++) verify_logits[i] = bf2f(tmp[i]);
    }
    return 0;
}
extern "C" int vx_spec_set_tracing(vx_spec *e, int enable) {
    VX_REQUIRE(e, "tracing: null engine");
    e->tracing = enable != 0;
    return 0;
}
extern "C" int vx_spec_last_trace_info(const vx_spec *e, vx_round_trace *info, int64_t *state_ids,
                                       uint32_t *stream_ids, uint32_t *rounds) {
    VX_REQUIRE(e && info, "trace: null argument");
    *info = vx_round_trace{};
    info->serial = e->serial;
    if (e->serial == 0) return 0;
    info->n = e->last_n;
    info->draft_k = e->last_k;
    info->vocab = e->target->cfg.vocab;
    info->temperature = e->last_temp;
    info->has_draft_logits = e->last_kept_draft ? 1 : 0;
    if (state_ids) memcpy(state_ids, e->last_ids.data(), e->last_ids.size() * 8);
    if (stream_ids) memcpy(stream_ids, e->last_streams.data(), e->last_streams.size() * 4);
    if (rounds) memcpy(rounds, e->last_rounds.data(), e->last_rounds.size() * 4);
    return 0;
}
extern "C" int vx_spec_last_trace_draft(const vx_spec *e, float *draft_logits, float *uniforms) {
    VX_REQUIRE(e && e->last_n > 0, "trace: no step yet");
    const int64_t n = e->last_n, D = e->last_k, V = e->target->cfg.vocab;
    if (draft_logits) {
        VX_REQUIRE(e->last_kept_draft, "trace: the last greedy round kept no draft logits (enable tracing)");
        std::vector<uint16_t> tmp((size_t)(D * n * V));
        VX_HIP(hipMemcpy(tmp.data(), e->d_dlog.p, tmp.size() * 2, hipMemcpyDeviceToHost));
        // device layout [D][n][V] -> [n][D][V]
        for (int64_t i = 0; i < D; i++)
            for (int64_t b = 0; b < n; b++) {
                const uint16_t *src = tmp.data() + (i * n + b) * V;
                float *dst = draft_logits + (b * D + i) * V;
                for (int64_t j = 0; j < V; j++) dst[j] = bf2f(src[j]);
            }
    }
    if (uniforms) {
        if (e->last_temp > 0.f)
            VX_HIP(hipMemcpy(uniforms, e->d_uni.p, (size_t)n * (D + 1) * 16, hipMemcpyDeviceToHost));
        else
            memset(uniforms, 0, (size_t)n * (D + 1) * 16);
    }
    return 0;
}
extern "C" int vx_spec_set_profiling(vx_spec *e, int enable) {
    VX_REQUIRE(e, "profiling: null engine");
    VX_REQUIRE(enable >= 0 && enable <= 2, "profiling: mode is 0, 1 (per kernel) or 2 (phases only)");
    e->profiling = enable;
    return 0;
}
extern "C" int vx_spec_last_profile(const vx_spec *e, vx_step_profile *out) {
    VX_REQUIRE(e && out, "profiling: null argument");
    VX_REQUIRE(e->profiling, "profiling: not enabled");
    *out = e->last_prof;
    return 0;
}
extern "C" void vx_spec_free(vx_spec *e, int64_t s) {
    if (!e || s < 0 || s >= (int64_t)e->states.size() || !e->states[s].live) return;
    SpecState &st = e->states[s];
    vx_pages_free(e->tp, st.target_blocks.data(), (int64_t)st.target_blocks.size());
    vx_pages_free(e->dp, st.draft_blocks.data(), (int64_t)st.draft_blocks.size());
    st = SpecState{};
}

extern "C" const char *vx_last_error(void) { return g_err.c_str(); }
extern "C" const char *vx_version(void) { return "velox_amd 0.1.0 (gfx950)"; }

// ===========================================================================
// the scheduler's engine binding (vx_sched_create)
// ===========================================================================
namespace {
struct SpecBinding {
    vx_spec *e;
    void *stream;
};
int sb_add_state(void *c, const uint32_t *prompt, int64_t len, int64_t cached, const uint32_t *tp,
                 const uint32_t *dp, int64_t reserve, uint32_t stream_id, float temperature, int64_t *out) {
    return vx_spec_add_state(((SpecBinding *)c)->e, prompt, len, cached, tp, dp, reserve, stream_id, temperature, out);
}
int sb_prefill_chunk(void *c, const int64_t *states, const int64_t *n_tokens, int64_t n) {
    auto *b = (SpecBinding *)c;
    return vx_spec_prefill_chunk(b->e, states, n_tokens, n, b->stream);
}
int sb_step(void *c, const int64_t *states, int64_t n, int64_t k, vx_round_outcome *outcomes, uint32_t *committed) {
    auto *b = (SpecBinding *)c;
    return vx_spec_step(b->e, states, n, k, -1, outcomes, committed, b->stream);
}
int64_t sb_state_pages(void *c, int64_t s, int which, uint32_t *out, int64_t cap) {
    return vx_spec_state_pages(((SpecBinding *)c)->e, s, which, out, cap);
}
void sb_free_state(void *c, int64_t s) { vx_spec_free(((SpecBinding *)c)->e, s); }
void sb_incref(void *c, int which, const uint32_t *pages, int64_t n) {
    vx_spec *e = ((SpecBinding *)c)->e;
    vx_pages_incref(which ? e->dp : e->tp, pages, n);
}
void sb_decref(void *c, int which, const uint32_t *pages, int64_t n) {
    vx_spec *e = ((SpecBinding *)c)->e;
    vx_pages_free(which ? e->dp : e->tp, pages, n);
}
void sb_release(void *c) { delete (SpecBinding *)c; }
}  // namespace

namespace vx {
int spec_sched_backend(vx_spec *e, void *stream, vx_sched_backend *out, void (**release)(void *)) {
    int64_t ps;
    VX_TRY(page_size_or_err(e, &ps));
    *out = vx_sched_backend{};
    out->ctx = new SpecBinding{e, stream};
    out->page_size = ps;
    out->add_state = sb_add_state;
    out->prefill_chunk = sb_prefill_chunk;
    out->step = sb_step;
    out->state_pages = sb_state_pages;
    out->free_state = sb_free_state;
    out->incref = sb_incref;
    out->decref = sb_decref;
    *release = sb_release;
    return 0;
}
}  // namespace vx
