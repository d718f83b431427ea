/*
 * velox_hip.h — C ABI of the MI355X (gfx950) speculative-decoding verify path.
 *
 * Drop-in boundary for the reference's Metal backend (Soflutionltd/velox,
 * src/paged/).  Conventions shared by every entry point:
 *   - returns 0 on success, non-zero on error; the message is available from
 *     vx_last_error() on the calling thread (the reference's anyhow::bail!);
 *   - tensors are caller-owned device pointers with explicit sizes, contiguous
 *     row-major, dtype given by a vx_dtype code; index tensors are uint32;
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream); work
 *     is enqueued asynchronously and ordered on that stream, like candle's
 *     command encoder;
 *   - entry points validate exactly what the reference validates, with the
 *     same failure conditions.
 * No torch or HIP types appear in the signatures.
 */
#ifndef VELOX_HIP_H
#define VELOX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { VX_F32 = 0, VX_F16 = 1, VX_BF16 = 2 } vx_dtype;

const char *vx_last_error(void);
const char *vx_version(void);

/* ======================================================================== */
/* Kernel-level operators (src/paged/metal_kernels.rs)                       */
/* ======================================================================== */

/* Replaces qmm_4bit (metal_kernels.rs:2069-2076; validation :2082-2130).
 * Y[M,N] = X[M,K] . deq(W)^T (+ bias), MLX int4 affine format:
 *   qweight [N, K/8] u32 (8 nibbles little-endian), scales/biases [N, K/g],
 *   w = q * scale + bias;  X, scales, biases, bias, Y share `dtype`.
 * bias may be NULL.  Split-K scratch comes from a library-owned per-stream
 * workspace allocated on first use. */
int vx_qmm_4bit(const void *x, const uint32_t *qweight, const void *scales, const void *biases,
                const void *bias, void *y, int64_t m, int64_t n, int64_t k, int64_t group_size,
                int dtype, void *stream);

/* vx_qmm_4bit for callers that cannot allocate device memory: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  No
 * counterpart in the reference.  Same arguments, validation, kernel plan and
 * results (bit for bit) as vx_qmm_4bit; it calls no hipMalloc / hipFree and
 * no allocating library routine.  Its split-K partials go to a static device
 * array of VX_QMM_NOALLOC_SCRATCH_BYTES per GPU (held until the process
 * ends); a shape whose plan needs more returns an error naming the sizes.
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (e.g. on two streams) race. */
#define VX_QMM_NOALLOC_SCRATCH_BYTES ((size_t)(16u << 20) + 65536u)
int vx_qmm_4bit_noalloc(const void *x, const uint32_t *qweight, const void *scales, const void *biases,
                        const void *bias, void *y, int64_t m, int64_t n, int64_t k, int64_t group_size,
                        int dtype, void *stream);

/* Epilogue variants used by the fused verify forward. */
typedef enum {
    VX_EPI_STORE = 0,    /* Y = round_T(acc)                                   */
    VX_EPI_RESIDUAL = 1, /* Y = round_T(R + round_T(acc)), R [M,N] in y_dtype   */
    VX_EPI_SWIGLU = 2    /* weights rows interleaved in 16-row blocks gate|up:
                            Y[m,f] = round_T(round_T(silu(g)) * u), Y [M, N/2] */
} vx_epilogue;

/* Extended int4 GEMM: X is f16 (any value representable in f16, optionally
 * holding X_true * 2^-x_shift), scales/biases f16 [N, K/g], accumulation in
 * f32, result rounded to `round_dtype` semantics and stored as `y_dtype`.
 * Requires group_size 64, K % 128 == 0, X 16-byte aligned, qweight rows
 * 16-byte aligned, scales/biases 4-byte aligned.  workspace (device, >= vx_qmm_workspace_size bytes, first 64 KiB zeroed
 * once by the caller and left zero by the kernel) may be NULL to use the
 * per-stream library workspace. */
int vx_qmm_4bit_ex(const void *x, const uint32_t *qweight, const void *scales,
                   const void *biases, void *y, const void *residual, int64_t m, int64_t n,
                   int64_t k, int64_t group_size, int x_shift, int round_dtype, int y_dtype,
                   int epilogue, void *workspace, size_t workspace_bytes, void *stream);
size_t vx_qmm_workspace_size(int64_t m, int64_t n, int64_t k);

/* Packed weights for the verify path (no reference counterpart: the
 * reference's Metal kernel reads MLX's row-major words, metal_kernels.rs
 * :418-479; the packed form holds the same values).  Per 32-row tile and
 * 128-wide k step, one 2304-byte block laid out for the 32x32x16 MFMA B
 * operand: 2048 bytes of nibbles (lane L: row L%32, k 16j + 8*(L/32) .. +7
 * for j < 8), then (scale, bias) of the step's two groups per row as f16.
 * N % 32 == 0, K % 128 == 0, group size 64.  vx_qmm_pack_4bit converts
 * device MLX tensors on `stream`; vx_qmm_4bit_packed is vx_qmm_4bit_ex over
 * packed weights (X 16-byte aligned). */
size_t vx_qmm_packed_size(int64_t n, int64_t k);
int vx_qmm_pack_4bit(const uint32_t *qweight, const void *scales, const void *biases, void *packed,
                     int64_t n, int64_t k, void *stream);
int vx_qmm_4bit_packed(const void *x, const void *packed, void *y, const void *residual, int64_t m,
                       int64_t n, int64_t k, int x_shift, int round_dtype, int y_dtype, int epilogue,
                       void *workspace, size_t workspace_bytes, void *stream);

/* Replaces paged_prefill_attention (metal_kernels.rs:1680-1690; validation
 * :1697-1745; kernel MSL :307-395) and, with tree_mask, extends it to tree
 * verification.  q [total_q, h_q, d]; k_pool/v_pool [P, h_kv, page_size, d];
 * block_table [n_seqs, max_blocks]; cu_seqlens [n_seqs+1]; seq_id_per_q
 * [total_q]; kv_offsets [n_seqs]; out [total_q, h_q, d].  tree_mask (device
 * uint64 [total_q] or NULL): row t of a sequence sees context positions
 * < kv_offset and tree slot kv_offset + j iff bit j is set; NULL keeps the
 * reference's causal rule (kv_len = kv_offset + t + 1).  q/k/v/out share
 * dtype.  Requires head_dim % 32 == 0, head_dim <= 256, h_q % h_kv == 0.
 * cu_seqlens, seq_id_per_q and kv_offsets are read back on the host (one
 * small copy and a stream synchronisation) to check the rows and size the
 * launch; KV-split partials use the per-stream library workspace. */
int vx_paged_attention(const void *q, const void *k_pool, const void *v_pool,
                       const uint32_t *block_table, const uint32_t *cu_seqlens,
                       const uint32_t *seq_id_per_q, const uint32_t *kv_offsets,
                       const uint64_t *tree_mask, void *out, int64_t total_q, int64_t n_seqs,
                       int64_t max_blocks, int64_t num_pages, int64_t h_q, int64_t h_kv,
                       int64_t head_dim, int64_t page_size, float scale, uint32_t sliding_window,
                       int dtype, void *stream);

/* Replaces paged_decode_attention (metal_kernels.rs:1227-1235; MSL :107-191):
 * one query row per sequence attending to kv_lens[n] positions. */
int vx_paged_decode_attention(const void *q, const void *k_pool, const void *v_pool,
                              const uint32_t *block_table, const uint32_t *kv_lens, void *out,
                              int64_t n, int64_t max_blocks, int64_t num_pages, int64_t h_q,
                              int64_t h_kv, int64_t head_dim, int64_t page_size, float scale,
                              uint32_t sliding_window, int dtype, void *stream);

/* Replaces batched_rope_decode (metal_kernels.rs:1414-1419; MSL :209-241):
 * in place on x [n, h, d] with per-row offsets[n] into cos/sin [max_pos, d/2]
 * (same dtype as x). */
int vx_rope_inplace(void *x, const void *cos_t, const void *sin_t, const uint32_t *offsets,
                    int64_t n, int64_t h, int64_t d, int64_t max_pos, int dtype, void *stream);

/* Replaces batched_scatter (metal_kernels.rs:1543-1548; MSL :251-279):
 * pool[page_ids[i], h, slots[i], :] = values[i, h, :]  (exact copy). */
int vx_kv_scatter(void *pool, const void *values, const uint32_t *page_ids,
                  const uint32_t *slots, int64_t n, int64_t num_pages, int64_t h,
                  int64_t page_size, int64_t d, int dtype, void *stream);

/* ======================================================================== */
/* Acceptance (src/paged/spec.rs:266-301) and its stochastic / tree          */
/* extensions.  Logits are [rows, vocab] in logits_dtype; outputs are device */
/* arrays.  `workspace` as for vx_qmm_4bit_ex (NULL = per-stream library     */
/* workspace).                                                               */
/* ======================================================================== */

/* argmax_slice (spec.rs:356-366) per row: strict '>', first index wins, NaN
 * never wins, all -inf/NaN -> 0. */
int vx_argmax_rows(const void *logits, uint32_t *out, int64_t rows, int64_t vocab,
                   int logits_dtype, void *stream);

/* Greedy accept + bonus (spec.rs:271-301) for `batch` sequences at once.
 * logits [batch, k+1, vocab]; candidates [batch, k];
 * accepted[b] = A; tokens[b, 0..A] = c[0..A) ++ argmax(T[A]). */
int vx_accept_greedy(const void *logits, const uint32_t *candidates, int32_t *accepted,
                     uint32_t *tokens, int64_t batch, int64_t k, int64_t vocab,
                     int logits_dtype, void *stream);

/* Stochastic acceptance (Leviathan et al. 2023 Alg. 1): p = softmax(lt/T),
 * q = softmax(ld/T); accept c_i iff u_acc < min(1, p(c_i)/q(c_i)); at the
 * first rejection draw from normalize(max(0, p - q)) with u_res; if all k
 * are accepted draw the bonus from p_k.  target [batch, k+1, vocab],
 * draft [batch, k, vocab], uniforms [batch, k+1, 4] f32 (slot 1 = u_acc,
 * slot 2 = u_res / bonus).  Reductions use a fixed order so decisions are
 * bit-identical to the host definition. */
int vx_accept_stochastic(const void *target_logits, const void *draft_logits,
                         const uint32_t *candidates, const float *uniforms, int32_t *accepted,
                         uint32_t *tokens, int64_t batch, int64_t k, int64_t vocab,
                         float temperature, int logits_dtype, void *workspace,
                         size_t workspace_bytes, void *stream);

/* Draft-token draw c[b,i] ~ softmax(ld[b,i]/T) with uniforms[b,i,0]. */
int vx_sample_rows(const void *logits, const float *uniforms, int64_t uniform_stride,
                   uint32_t *out, int64_t rows, int64_t vocab, float temperature,
                   int logits_dtype, void *workspace, size_t workspace_bytes, void *stream);

/* Greedy tree acceptance: node 0 is the root (the last committed token);
 * parents [r] (host array, parents[j] < j); node_tokens [batch, r];
 * logits [batch, r, vocab].  accepted[b] = path length A; path[b, 0..A]
 * node indices; tokens[b, 0..A] = tokens of path[1..A] ++ bonus. */
int vx_accept_tree(const void *logits, const int32_t *parents, const uint32_t *node_tokens,
                   int32_t *accepted, int32_t *path, uint32_t *tokens, int64_t batch, int64_t r,
                   int64_t vocab, int logits_dtype, void *stream);

/* ======================================================================== */
/* Engine level: PagedKvCache (pages.rs), PagedQwen3 (qwen3.rs) and          */
/* SpecEngine (spec.rs).                                                     */
/* ======================================================================== */

typedef struct vx_pages vx_pages;
typedef struct vx_model vx_model;
typedef struct vx_spec vx_spec;

/* PagedKvConfig + PagedKvCache::new (pages.rs:33-40, :93-136): per-layer K
 * and V pools [num_pages, kv_heads, page_size, head_dim] in kv_dtype,
 * zero-initialised; free list pops page 0 first. */
int vx_pages_create(int64_t layers, int64_t kv_heads, int64_t head_dim, int64_t page_size,
                    int64_t num_pages, int kv_dtype, vx_pages **out);
void vx_pages_destroy(vx_pages *p);
/* PagedKvCache::alloc (pages.rs:173-186): all-or-nothing; returns non-zero
 * ("not enough free pages") without taking any page. */
int vx_pages_alloc(vx_pages *p, int64_t n, uint32_t *out_pages);
/* PagedKvCache::incref_pages / free_pages (pages.rs:192-234). */
void vx_pages_incref(vx_pages *p, const uint32_t *pages, int64_t n);
void vx_pages_free(vx_pages *p, const uint32_t *pages, int64_t n);
int64_t vx_pages_num_free(const vx_pages *p);
uint32_t vx_pages_refcount(const vx_pages *p, uint32_t page);
/* layer_k_pool / layer_v_pool (pages.rs:248-254): device pointer. */
void *vx_pages_pool(vx_pages *p, int64_t layer, int kv);

/* Qwen3Config (qwen3.rs:31-60) subset used by the path. */
typedef struct {
    int64_t vocab, hidden, inter, layers, n_heads, n_kv_heads, head_dim;
    int64_t max_pos, group_size;
    double rope_theta, rms_eps;
} vx_qwen3_config;

/* One MLX int4 linear from host memory (qwen3.rs:204-211): qweight u32
 * [N, K/8]; scales, biases f16 [N, K/g]. */
typedef struct {
    const uint32_t *qweight;
    const uint16_t *scales, *biases;
} vx_qlinear_host;

typedef struct {
    const uint16_t *ln1, *ln2, *q_norm, *k_norm; /* f16 [hidden] / [head_dim] */
    vx_qlinear_host q, k, v, o, gate, up, down;
} vx_layer_host;

typedef struct {
    const uint16_t *embed; /* f16 [vocab, hidden] */
    const vx_layer_host *layers;
    const uint16_t *norm;
    vx_qlinear_host lm_head;
} vx_weights_host;

/* PagedQwen3::load (qwen3.rs:954-986) from host arrays.  Float tensors are
 * converted to the model dtype (bf16) the way candle's VarBuilder converts
 * them; KV pages attached later must use kv_dtype f16 or bf16. */
int vx_model_create(const vx_qwen3_config *cfg, const vx_weights_host *w, int64_t n_layers,
                    vx_model **out);
void vx_model_destroy(vx_model *m);

/* Tree-path KV compaction.  No counterpart in the reference (its spec loop
 * is a chain); tree verification (vx_forward with tree_parents) writes node j
 * of each sequence at position kv_offset + j, and after vx_accept_tree the
 * accepted path must sit at consecutive positions: for d = 1..accepted[b],
 * position kv_offsets[b] + d receives, in every layer, K and V and kv head,
 * the row of node path[b, d] (position kv_offsets[b] + path[b, d]); the root
 * (d = 0) stays.  Every destination receives its source's value from before
 * the call.  block_tables [n_seqs, max_blocks] u32, kv_offsets [n_seqs] u32,
 * accepted [n_seqs] i32, path [n_seqs, r] i32: device arrays, as
 * vx_accept_tree writes them.  r <= 64. */
int vx_kv_compact_path(vx_pages *pages, const uint32_t *block_tables, int64_t max_blocks,
                       const uint32_t *kv_offsets, const int32_t *accepted, const int32_t *path,
                       int64_t n_seqs, int64_t r, void *stream);

/* SeqSlice (qwen3.rs:254-263): block_table is a host array. */
typedef struct {
    int64_t new_tokens, kv_offset;
    const uint32_t *block_table;
    int64_t n_blocks;
} vx_seq_slice;

/* PagedQwen3::forward_all (qwen3.rs:1023-1036) when all_rows != 0, else
 * PagedQwen3::forward (:994-1017, last row per sequence).  input_ids is a
 * host array [sum new_tokens]; logits is a device array [rows, vocab] in
 * bf16.  tree_parents (host, may be NULL): every sequence carries the same
 * R-node tree (R = new_tokens <= 64), node j written at slot kv_offset + j,
 * rotated at kv_offset + depth(j), attending to the context and its
 * ancestors. */
int vx_forward(vx_model *m, vx_pages *pages, const uint32_t *input_ids,
               const vx_seq_slice *seqs, int64_t n_seqs, int all_rows,
               const int32_t *tree_parents, void *logits, void *stream);

/* SpecEngine::new (spec.rs:70-94): rejects vocab / page-size mismatch.
 * temperature 0 = greedy (the reference's mode); > 0 = stochastic acceptance
 * with Philox uniforms keyed by sample_seed.  fix_draft_hole = 0 reproduces
 * spec.rs exactly (c[D-1] never fed to the draft). */
int vx_spec_create(vx_model *target, vx_pages *target_pages, vx_model *draft,
                   vx_pages *draft_pages, float temperature, uint64_t sample_seed,
                   int fix_draft_hole, vx_spec **out);
void vx_spec_destroy(vx_spec *e);

/* SpecEngine::prefill (spec.rs:131-182) for n prompts (host arrays), batched;
 * states are numbered 0..n-1 in the returned order (the engine keeps them). */
int vx_spec_prefill(vx_spec *e, const uint32_t *const *prompts, const int64_t *lens, int64_t n,
                    int64_t *out_first_state);

/* RoundOutcome (spec.rs:327-335) for one state. */
typedef struct {
    int32_t accepted;
    int32_t n_committed;
    int32_t stop;
} vx_round_outcome;

/* SpecEngine::step (spec.rs:186-316) over n states at once (one batched
 * draft forward per draft position, one batched verify, one acceptance
 * launch).  committed: host [n, draft_k+1] (row b holds outcome[b].n_committed
 * tokens).  eos < 0: none.  draft_k == 0 is an error (spec.rs:192-194). */
int vx_spec_step(vx_spec *e, const int64_t *state_ids, int64_t n, int64_t draft_k, int64_t eos,
                 vx_round_outcome *outcomes, uint32_t *committed, void *stream);

/* SpecState accessors (spec.rs:110-124). */
int64_t vx_spec_state_kv_len(const vx_spec *e, int64_t state);
int64_t vx_spec_state_num_tokens(const vx_spec *e, int64_t state);
int vx_spec_state_tokens(const vx_spec *e, int64_t state, uint32_t *out, int64_t cap);
/* Debug/trace copies of the last step (host): candidates [n, k], verify
 * logits [n, k+1, vocab] as f32. */
int vx_spec_last_trace(const vx_spec *e, uint32_t *candidates, float *verify_logits);

/* Round trace (no reference counterpart: the reference's spec test reads
 * only committed tokens, tests/spec_decode.rs:182-213).  It lets a checker
 * re-derive every decision of the last vx_spec_step from the GPU's own
 * inputs.  With tracing enabled, greedy rounds keep the logits of every draft
 * step (stochastic rounds always do); it costs n * k * vocab * 2 bytes. */
typedef struct {
    int64_t n, draft_k, vocab;
    float temperature;          /* of the last round; 0 = greedy */
    int32_t has_draft_logits;   /* draft logits of every step are available */
    uint64_t serial;            /* number of rounds run by the engine (0: none) */
} vx_round_trace;
int vx_spec_set_tracing(vx_spec *e, int enable);
/* state_ids [n], stream_ids [n], rounds [n] (the Philox counter words the
 * round's uniforms were drawn with); each may be NULL. */
int vx_spec_last_trace_info(const vx_spec *e, vx_round_trace *info, int64_t *state_ids,
                            uint32_t *stream_ids, uint32_t *rounds);
/* draft_logits [n, k, vocab] as f32 (sequence-major; the values the draft
 * argmax or draw read), uniforms [n, k+1, 4] (zeros for a greedy round);
 * each may be NULL. */
int vx_spec_last_trace_draft(const vx_spec *e, float *draft_logits, float *uniforms);

/* Per-kernel HIP-event timing of a step (no reference counterpart: the
 * reference's only timing is Instant around calls, tests/spec_decode.rs).
 * Classes: 0 = int4 GEMM, 1 = paged attention, 2 = other.  Bytes are
 * algorithmic (each weight / KV / activation byte counted once). */
typedef struct {
    double draft_ms, verify_ms, accept_ms;
    double verify_kernel_ms[3], verify_kernel_bytes[3];
    int64_t verify_kernel_launches[3];
    double draft_kernel_ms[3], draft_kernel_bytes[3];
    int64_t draft_kernel_launches[3];
} vx_step_profile;
/* enable: 0 off; 1 events around every kernel and at the phase boundaries
 * (each event pair also brackets its kernel's dispatch gap); 2 phase
 * boundaries only (draft / verify / accept ms of an undisturbed round). */
int vx_spec_set_profiling(vx_spec *e, int enable);
int vx_spec_last_profile(const vx_spec *e, vx_step_profile *out);

/* SpecEngine::free (spec.rs:320-323). */
void vx_spec_free(vx_spec *e, int64_t state);

/* Continuous batching support (the reference's scheduler admits a request,
 * scheduler.rs:221-296, then prefills it inside its packed step, :299-368).
 *
 * vx_spec_add_state creates a state for prompt[0, len) without running
 * anything.  Its first cached_tokens positions (a multiple of page_size,
 * at most len - 1) are already in KV, in target_pages / draft_pages
 * [cached_tokens / page_size]; the state takes over one reference to each
 * (vx_spec_free releases it).  Pages covering max(reserve_tokens, len - 1)
 * positions are allocated now, all or nothing over both pools ("not enough
 * free pages" leaves everything as it was).  stream_id keys the state's
 * Philox uniforms (rounds count from 0); temperature < 0 takes the engine's.
 * The state is ready for vx_spec_step once prompt[..len-1] is in KV: at
 * once when cached_tokens == len - 1, else after vx_spec_prefill_chunk has
 * fed the rest.  Freed state numbers are reused. */
int vx_spec_add_state(vx_spec *e, const uint32_t *prompt, int64_t len, int64_t cached_tokens,
                      const uint32_t *target_pages, const uint32_t *draft_pages, int64_t reserve_tokens,
                      uint32_t stream_id, float temperature, int64_t *out_state);
/* One batched forward of both models over the next n_tokens[b] prompt
 * tokens of each listed state (at positions kv_len .. kv_len + n_tokens - 1,
 * never past len - 2); logits are discarded as in spec.rs:172-173. */
int vx_spec_prefill_chunk(vx_spec *e, const int64_t *state_ids, const int64_t *n_tokens, int64_t n,
                          void *stream);
/* Block table of a state (which: 0 target, 1 draft); returns its length and
 * copies up to cap entries; -1 for an unknown state. */
int64_t vx_spec_state_pages(const vx_spec *e, int64_t state, int which, uint32_t *out, int64_t cap);

/* ------------------------------------------------------------------------
 * Continuous-batching speculative scheduler: BatchScheduler
 * (scheduler.rs:37-534) with spec rounds in place of its one-token decode,
 * and PrefixCache (prefix_cache.rs:1-230) over target + draft page pairs.
 *
 * Each vx_sched_step:
 *  1. admits waiting requests in FCFS order while fewer than
 *     max_running_requests run: a prefix-cache lookup (whole pages of
 *     prompt[..len-1]), then vx_spec_add_state reserving len + max_new +
 *     draft_k positions; a request that does not fit stays at the head of
 *     the queue (scheduler.rs:221-296).  A request whose next uncached
 *     prompt page another running request is still prefilling waits, so it
 *     shares that page instead of computing it again.
 *  2. walks the running requests by id under max_batch_tokens
 *     (scheduler.rs:299-337): a prefilling request takes the rest of its
 *     prompt, cut to the budget left (a chunk); a decoding request costs
 *     draft_k + 1 verify rows and is deferred when they do not fit.  The
 *     first request always runs.
 *  3. runs one vx_spec_prefill_chunk for the chunks, registers every prompt
 *     page completed by it in the prefix cache, and runs vx_spec_step for
 *     the decoding requests (one call per distinct temperature).
 *  4. appends committed tokens, stops at an EOS id ("stop") or max_new
 *     tokens ("length"), truncating the round's surplus, and frees the
 *     finished requests' states (scheduler.rs:369-500).
 * ---------------------------------------------------------------------- */
typedef struct vx_sched vx_sched;

typedef struct {
    int64_t max_running_requests;   /* scheduler.rs:37-59 default 64 */
    int64_t max_batch_tokens;       /* default 512 */
    int64_t prefix_cache_capacity;  /* cached page pairs; 0 disables; default 256 */
    int64_t draft_k;                /* draft tokens per round */
} vx_sched_config;

/* SchedulerStats (scheduler.rs:94-105) plus the spec counters. */
typedef struct {
    uint64_t steps, tokens_generated, requests_completed, requests_aborted;
    uint64_t last_batch_size, last_step_us;
    uint64_t prefix_cache_hits, prefix_cache_misses, prefix_tokens_skipped;
    uint64_t rounds, draft_tokens_proposed, draft_tokens_accepted, prefill_tokens;
} vx_sched_stats;

/* The engine the scheduler drives.  vx_sched_create binds it to a vx_spec
 * and its two page pools; vx_sched_create_with_backend takes any engine
 * with these semantics (which: 0 target pool, 1 draft pool):
 *  add_state / prefill_chunk / step / state_pages / free_state as the
 *  vx_spec_* calls above (step with eos -1, on the scheduler's stream);
 *  incref / decref as vx_pages_incref / vx_pages_free on a pool. */
typedef struct {
    void *ctx;
    int64_t page_size;
    int (*add_state)(void *ctx, const uint32_t *prompt, int64_t len, int64_t cached_tokens,
                     const uint32_t *target_pages, const uint32_t *draft_pages, int64_t reserve_tokens,
                     uint32_t stream_id, float temperature, int64_t *out_state);
    int (*prefill_chunk)(void *ctx, const int64_t *states, const int64_t *n_tokens, int64_t n);
    int (*step)(void *ctx, const int64_t *states, int64_t n, int64_t draft_k, vx_round_outcome *outcomes,
                uint32_t *committed);
    int64_t (*state_pages)(void *ctx, int64_t state, int which, uint32_t *out, int64_t cap);
    void (*free_state)(void *ctx, int64_t state);
    void (*incref)(void *ctx, int which, const uint32_t *pages, int64_t n);
    void (*decref)(void *ctx, int which, const uint32_t *pages, int64_t n);
} vx_sched_backend;

/* BatchScheduler::new (scheduler.rs:108-137).  eos_ids: host array (the
 * reference's eos_token_ids).  The engine must outlive the scheduler. */
int vx_sched_create(vx_spec *engine, const vx_sched_config *cfg, const uint32_t *eos_ids, int64_t n_eos,
                    void *stream, vx_sched **out);
int vx_sched_create_with_backend(const vx_sched_backend *backend, const vx_sched_config *cfg,
                                 const uint32_t *eos_ids, int64_t n_eos, vx_sched **out);
/* Frees every live state and clears the prefix cache (PrefixCache::clear). */
void vx_sched_destroy(vx_sched *s);
/* BatchScheduler::submit (scheduler.rs:147-185) for a tokenised prompt:
 * "Empty prompt" for len 0; a spec round needs len >= 2.  max_new_tokens
 * is raised to 1 as in the reference.  temperature <= 1e-7 is greedy
 * (scheduler.rs:555-559).  stream < 0 keys the Philox uniforms by the
 * request id, so a request's samples do not depend on its batch mates.
 * Returns ids 1, 2, 3, ... (RequestId, request.rs:11-21). */
int vx_sched_submit(vx_sched *s, const uint32_t *prompt, int64_t len, int64_t max_new_tokens, float temperature,
                    int64_t stream, int64_t *out_id);
/* One scheduler step (admit + BatchScheduler::step); *out_tokens = the new
 * tokens it fed to the models (0 when idle). */
int vx_sched_step(vx_sched *s, int64_t *out_tokens);
/* Request state: tokens generated so far (up to cap copied), status
 * 0 waiting / 1 running / 2 finished / 3 aborted, finish reason 0 none /
 * 1 stop / 2 length / 3 cancelled. */
int vx_sched_poll(vx_sched *s, int64_t id, uint32_t *tokens, int64_t cap, int64_t *n_tokens, int *status,
                  int *finish_reason);
/* Cancel a waiting or running request (the reference's client disconnect,
 * scheduler.rs:441-453); its pages go back at once. */
int vx_sched_abort(vx_sched *s, int64_t id);
/* Forget a finished or aborted request's record. */
int vx_sched_release(vx_sched *s, int64_t id);
int vx_sched_get_stats(vx_sched *s, vx_sched_stats *out);
/* Requests waiting / running; page pairs held by the prefix cache. */
int64_t vx_sched_num_waiting(vx_sched *s);
int64_t vx_sched_num_running(vx_sched *s);
int64_t vx_sched_cache_pages(vx_sched *s);

#ifdef __cplusplus
}
#endif
#endif
