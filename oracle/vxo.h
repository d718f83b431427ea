/*
 * vxo — CPU oracle for the speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product path (velox_amd/) never links,
 * loads or calls it.
 *
 * Every function restates the reference's algorithm in plain C with the
 * reference's loop order and rounding points; the citation next to each
 * declaration names the reference file:line it follows.  Floating point is
 * compiled with -ffp-contract=off so that a*b+c stays two IEEE roundings, as
 * in the reference's Rust (Rust never contracts).
 *
 * Tensors are float arrays whose values are already rounded to the storage
 * dtype they stand for (f16 / bf16 / f32); `dtype` arguments name where a
 * result is rounded back to storage precision, as the reference does when a
 * candle op returns a tensor of dtype T.
 *
 * Parity status (what pins each function; tests/test_oracle*.py):
 *   f32/f16/bf16 rounding     closed form vs numpy casts (test_round_to_dtypes)
 *   philox4x32_10, u01        Random123 known answers + rocRAND fixture
 *                             (test_philox_*), uniform layout (test_uniforms_layout)
 *   expf                      <= 2 ulp of libm double (test_deterministic_exp_accuracy)
 *   pack/unpack int4          dyn_quant.rs:205-218 known answer (test_pack_known_answer)
 *   qmm_4bit                  dense X.deq(W)^T, group sizes + bias, all-zero codes
 *                             (y = sum_g b_g sum x), one group, M=1 == row of M>1
 *   paged_attention           dense softmax (causal, tree, window); shuffled block
 *                             table invariance; chain tree == causal; kv_len 1 -> V
 *   rope_tables / rope_apply  closed form (f32 argument) / complex rotation
 *   kv_scatter                byte-exact copy
 *   argmax, accept_greedy     spec.rs:271-301, :356-366 cases (first index, NaN)
 *   row_softmax_stats         float64 log-sum-exp at V = 151936 with the maximum in
 *                             the first, a middle, the last and the partial chunk
 *                             (test_oracle_sampler.py)
 *   sample_residual           float64 inverse CDF at V = 8193 / 20000 / 151936 with
 *                             mass on both sides of every 256 / 8192 boundary;
 *                             chi-square of draws straddling them
 *   accept_stochastic, sample_draft
 *                             p == q accepts everything; emitted tokens follow p
 *                             (chi-square); no reference counterpart exists
 *   accept_tree, tree_masks   brute-force walks on small trees
 *   forward (model)           float64 dense Qwen3 (F32 oracle within 1e-4);
 *                             batched == per sequence (bit-exact)
 *   spec engine               spec greedy == target-only greedy; draft-KV hole
 *                             quirk and fix; error and capacity cases
 *   pages                     pages.rs:295-301 total_bytes, LIFO, all-or-nothing
 *   rmsnorm, silu             formula pinned through the model checks above; the
 *                             bf16 rounding points inside candle's RmsNorm / SiLU
 *                             are "parity unpinned" (candle 0.10.2 is not in the
 *                             reference tree and no reference test fixes them)
 */
#ifndef VXO_H
#define VXO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { VXO_F32 = 0, VXO_F16 = 1, VXO_BF16 = 2 };

/* ---- storage rounding (IEEE round-to-nearest-even) ---------------------- */
uint16_t vxo_f32_to_f16(float x);
float vxo_f16_to_f32(uint16_t h);
uint16_t vxo_f32_to_bf16(float x);
float vxo_bf16_to_f32(uint16_t h);
float vxo_round(float x, int dtype);
void vxo_round_array(float *x, int64_t n, int dtype);

/* ---- Philox4x32-10 (Salmon et al., SC'11) and derived uniforms ---------- */
void vxo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* u = (x >> 8) * 2^-24, in [0, 1) */
float vxo_u01(uint32_t x);
/* Spec-decode uniforms: out[b][i][0..3] = u01(philox(key=(seed_lo, seed_hi),
 * ctr=(stream0 + b, round, i, 0))) for b < batch, i < k + 1.
 * Slot 0: draft-token sampling, 1: accept test, 2: residual / bonus draw. */
void vxo_spec_uniforms(uint64_t seed, uint32_t stream0, uint32_t round, int64_t batch,
                       int64_t k, float *out);

/* Deterministic single-precision exp used by the stochastic acceptance (the
 * reference has no stochastic acceptance; this is the path's own definition,
 * shared bit-for-bit with the device code). */
float vxo_expf(float x);

/* ---- MLX int4 g64 packing (src/paged/dyn_quant.rs:125-151) -------------- */
void vxo_pack_int4(const uint32_t *codes, int64_t n, int64_t k, uint32_t *packed);
void vxo_unpack_int4(const uint32_t *packed, int64_t n, int64_t k, uint32_t *codes);

/* ---- qmm_4bit_cpu (src/paged/metal_kernels.rs:2325-2367) ----------------
 * y[m, n] (zero-initialised, then accumulated in the reference's loop order
 * n -> group -> packed word -> nibble -> row).  threads > 1 splits the n loop
 * (each output element keeps its sequential accumulation order). */
int vxo_qmm_4bit(const float *x, const uint32_t *qweight, const float *scales,
                 const float *biases, const float *bias_or_null, float *y, int64_t m,
                 int64_t n, int64_t k, int64_t group_size, int threads);

/* ---- paged attention ------------------------------------------------------
 * Online softmax of paged_decode_attention_cpu (metal_kernels.rs:2374-2438)
 * with the per-row visibility of paged_prefill_attention (MSL :307-395):
 *   seq = row's sequence, t = row - cu_seqlens[seq], off = kv_offsets[seq],
 *   tree_mask == NULL : key position p visible iff p <= off + t   (causal)
 *   tree_mask != NULL : p < off visible; p = off + j (j < 64) visible iff
 *                       bit j of tree_mask[row]; nothing else visible.
 * Sliding window (0 = off) hides p < (off + t + 1) - W.  Layout:
 *   q [total_q, h_q, d], pools [P, h_kv, page_size, d],
 *   block_table [n_seqs, max_blocks], out [total_q, h_q, d] (f32, unrounded). */
int vxo_paged_attention(const float *q, const float *k_pool, const float *v_pool,
                        const uint32_t *block_table, int64_t max_blocks,
                        const uint32_t *cu_seqlens, const uint32_t *kv_offsets,
                        int64_t n_seqs, const uint64_t *tree_mask, int64_t total_q,
                        int64_t h_q, int64_t h_kv, int64_t head_dim, int64_t page_size,
                        float scale, uint32_t sliding_window, float *out);

/* ---- RoPE (qwen3.rs:278-295 tables; MSL :209-241 apply) ------------------ */
void vxo_rope_tables(int64_t max_pos, int64_t head_dim, double theta, float *cos_t,
                     float *sin_t);
/* in place on x [n, h, d]; pos[n] per row; tables [max_pos, d/2] */
void vxo_rope_apply(float *x, const float *cos_t, const float *sin_t, const uint32_t *pos,
                    int64_t n, int64_t h, int64_t d, int dtype);
/* batched_scatter (MSL :251-279): pool[page_ids[n], h, slots[n], :] = values[n, h, :] */
void vxo_kv_scatter(float *pool, const float *values, const uint32_t *page_ids,
                    const uint32_t *slots, int64_t n, int64_t h, int64_t s, int64_t d);

/* ---- candle ops on the path (third-party; rounding points unpinned) ----- */
void vxo_rmsnorm(const float *x, const float *w, float *y, int64_t rows, int64_t dim,
                 float eps, int dtype);
float vxo_silu(float x);

/* ---- acceptance ---------------------------------------------------------- */
/* argmax_slice (spec.rs:356-366): strict '>', first index wins, NaN never wins */
uint32_t vxo_argmax(const float *v, int64_t n);
/* Greedy accept + bonus (spec.rs:271-301), batched over sequences.
 * logits [batch, k+1, vocab]; candidates [batch, k];
 * accepted[b] = A, tokens[b, 0..A] = c[0..A) ++ [bonus]. */
void vxo_accept_greedy(const float *logits, int64_t vocab, const uint32_t *candidates,
                       int64_t batch, int64_t k, int32_t *accepted, uint32_t *tokens);

/* Row softmax statistics with the fixed reduction structure shared with the
 * device kernels: chunks of VXO_SM_CHUNK elements, 256 strided thread partials
 * per chunk folded by a stride-halving tree, chunks combined in index order. */
#define VXO_SM_CHUNK 8192
#define VXO_SM_THREADS 256
#define VXO_SM_SUB 256
void vxo_row_softmax_stats(const float *row, int64_t vocab, float inv_t, float *m_out,
                           float *z_out);
/* Inverse-CDF draw from r_j = max(0, p_j - q_j) (q == NULL: r_j = p_j), with
 * p_j = e((lt_j - mt) * inv_t) / zt; hierarchical prefix order chunk ->
 * 256-element sub-chunk -> element. */
uint32_t vxo_sample_residual(const float *lt, float mt, float zt, const float *ld, float md,
                             float zd, int64_t vocab, float inv_t, float u);
/* Stochastic acceptance (Leviathan et al. 2023 Alg. 1; not in the reference).
 * target [batch, k+1, vocab], draft [batch, k, vocab], candidates [batch, k],
 * uniforms [batch, k+1, 4]. */
void vxo_accept_stochastic(const float *target_logits, const float *draft_logits,
                           const uint32_t *candidates, const float *uniforms, int64_t batch,
                           int64_t k, int64_t vocab, float inv_t, int32_t *accepted,
                           uint32_t *tokens);
/* Draw candidates: c[b, i] = sample(q_{b,i}, uniforms[b, i, 0]). */
void vxo_sample_draft(const float *draft_logits, const float *uniforms, int64_t batch,
                      int64_t k, int64_t vocab, float inv_t, uint32_t *candidates);
/* Greedy tree acceptance: node 0 is the root; parents[j] < j.  logits
 * [batch, R, vocab]; node_tokens [batch, R].  path[b, 0..A] node indices
 * (path[b,0] = 0); tokens[b, 0..A] = node tokens of path[1..A] ++ [bonus]. */
void vxo_accept_tree(const float *logits, const int32_t *parents, const uint32_t *node_tokens,
                     int64_t batch, int64_t r, int64_t vocab, int32_t *accepted,
                     int32_t *path, uint32_t *tokens);
/* Ancestor masks (bit j of mask[i] set iff j is i or an ancestor of i) and depths. */
void vxo_tree_masks(const int32_t *parents, int64_t r, uint64_t *masks, int32_t *depth);

/* ---- model, pages, spec engine ------------------------------------------ */
typedef struct {
    int64_t vocab, hidden, inter, layers, n_heads, n_kv_heads, head_dim;
    int64_t max_pos, group_size;
    double rope_theta, rms_eps;
    int dtype; /* T: activations, KV pools, logits (reference: vb.dtype()) */
} vxo_config;

typedef struct {
    const uint32_t *qweight; /* [N, K/8] */
    const float *scales;     /* [N, K/g], T-rounded */
    const float *biases;     /* [N, K/g], T-rounded */
} vxo_qlinear;

typedef struct {
    const float *ln1, *ln2, *q_norm, *k_norm; /* T-rounded */
    vxo_qlinear q, k, v, o, gate, up, down;
} vxo_layer;

typedef struct {
    const float *embed; /* [vocab, hidden], T-rounded */
    const vxo_layer *layers;
    const float *norm;
    vxo_qlinear lm_head;
} vxo_weights;

typedef struct vxo_model vxo_model;
typedef struct vxo_pages vxo_pages;

vxo_model *vxo_model_create(const vxo_config *cfg, const vxo_weights *w, int threads);
void vxo_model_destroy(vxo_model *m);

/* pages.rs:82-234: per-layer pools [P, h_kv, page_size, d] zero-initialised,
 * LIFO free list with page 0 first, refcounts, all-or-nothing alloc. */
vxo_pages *vxo_pages_create(int64_t layers, int64_t kv_heads, int64_t head_dim,
                            int64_t page_size, int64_t num_pages);
void vxo_pages_destroy(vxo_pages *p);
int vxo_pages_alloc(vxo_pages *p, int64_t n, uint32_t *out); /* 0 ok, -1 not enough */
void vxo_pages_free(vxo_pages *p, const uint32_t *pages, int64_t n);
int64_t vxo_pages_num_free(const vxo_pages *p);
float *vxo_pages_pool(vxo_pages *p, int64_t layer, int kv); /* kv: 0 = K, 1 = V */

typedef struct {
    int64_t new_tokens, kv_offset;
    const uint32_t *block_table;
    int64_t n_blocks;
} vxo_seq;

/* PagedQwen3::forward_all (qwen3.rs:1023-1036) when all_rows != 0, else
 * PagedQwen3::forward (:994-1017: last row per sequence).  With
 * tree_parents != NULL every sequence carries the same R = new_tokens node
 * tree: node j is written at slot kv_offset + j, rotated at position
 * kv_offset + depth(j) and attends to the context plus its ancestors. */
int vxo_forward(vxo_model *m, vxo_pages *pages, const uint32_t *ids, const vxo_seq *seqs,
                int64_t n_seqs, int all_rows, const int32_t *tree_parents, float *logits);

/* SpecEngine (spec.rs). */
typedef struct {
    uint32_t *target_blocks, *draft_blocks;
    int64_t n_target_blocks, n_draft_blocks;
    int64_t kv_len;
    uint32_t last_token;
    uint32_t *tokens;
    int64_t n_tokens;
    uint32_t stream_id, round;
} vxo_spec_state;

typedef struct {
    vxo_model *target, *draft;
    vxo_pages *target_pages, *draft_pages;
    float temperature;    /* 0 => greedy (the reference's only mode) */
    uint64_t sample_seed; /* Philox key for stochastic mode */
    int fix_draft_hole;   /* 0 = reproduce spec.rs (c[D-1] never fed to the draft) */
} vxo_spec;

/* prefill (spec.rs:131-182) for n prompts, batched into one forward per model. */
int vxo_spec_prefill(vxo_spec *e, const uint32_t *const *prompts, const int64_t *lens,
                     int64_t n, vxo_spec_state *states);
/* The state prefill would produce for prompt[0, len) (kv_len = len - 1,
 * pages for len positions in both pools) without running the models: the
 * caller fills the KV pages (e.g. copied from another implementation's
 * prefill of the same prompt) before stepping. */
int vxo_spec_adopt(vxo_spec *e, const uint32_t *prompt, int64_t len, vxo_spec_state *s);
/* step (spec.rs:186-316) for n states; committed[b, 0..accepted[b]] written to
 * committed (stride draft_k + 1); stop[b] as spec.rs:306-309 (eos < 0: none).
 * Optional trace outputs (NULL to skip): candidates [n, k],
 * verify_logits [n, k+1, vocab]. */
int vxo_spec_step(vxo_spec *e, vxo_spec_state *states, int64_t n, int64_t draft_k,
                  int64_t eos, int32_t *accepted, uint32_t *committed, int32_t *stop,
                  uint32_t *trace_candidates, float *trace_logits);
void vxo_spec_free(vxo_spec *e, vxo_spec_state *s);

const char *vxo_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
