/*
 * dspark_amd.h - C ABI of the MI355X (gfx950) DSpark attention hot path.
 *
 * Every pointer is a device pointer the caller owns (torch tensors in the
 * Python host layer); the library allocates nothing.  Every call is
 * asynchronous on `stream` (a hipStream_t) and never synchronises the host.
 * Return value: 0 on success, -1 for an invalid argument (nothing was
 * launched), -2 for a HIP launch failure; dspark_last_error() then returns a
 * thread-local message.
 *
 * Attention entry points are specialised to the Qwen3-0.6B geometry:
 * 16 query heads, 8 KV heads, head dim 128, bf16 in and out, FP32 softmax.
 * K/V token rows are [8][128] bf16 (2 KiB); query/output rows [16][128].
 */
#ifndef DSPARK_AMD_H
#define DSPARK_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Thread-local message for the last failing call on this thread. */
const char* dspark_last_error(void);

/* ABI revision of this header (currently 7). */
int dspark_abi_version(void);

/*
 * Measurement utility, no reference counterpart: reads `bytes` (a multiple
 * of 16) of device memory at `src` with `workgroups` workgroups of 256
 * threads, each streaming its own contiguous slice with 16-byte loads
 * (nontemporal = 1: non-temporal cache policy), and writes one uint32
 * checksum per workgroup to out[workgroups].  Its rate is the streaming-read
 * ceiling the attention kernels' bandwidth is compared with.
 */
int dspark_stream_read(const void* src, int64_t bytes, int nontemporal, int workgroups, void* out, void* stream);

/*
 * Measurement utility, no reference counterpart: the read bandwidth each XCD
 * gets from a region.  `workgroups` (a multiple of 8) workgroups of 256
 * threads each stream their own contiguous slice of `bytes` at `src` with
 * non-temporal 16-byte loads; workgroup w (which runs on XCD w mod 8)
 * writes stamps[3w] = start and stamps[3w+1] = end (a 100 MHz constant
 * clock) and stamps[3w+2] = its XCD id (low 32 bits) with the slice's
 * checksum (high 32 bits).  The caller derives per-XCD speeds, e.g. for the
 * xcd-weighted plans of the varlen / verify work lists.
 */
int dspark_xcd_read_stamps(const void* src, int64_t bytes, int workgroups, void* stamps, void* stream);

/*
 * Bytes of split-K workspace needed by an attention call.  Layout: FP32
 * partial outputs, then FP32 (max, sum) pairs, for `n` partial slots of 8 KV
 * heads x `row_tiles` 16-row tiles (row_tiles = ceil(max_q/8) for
 * varlen/verify, max blocks per request for draft), where
 *   n = ceil(key_rows_bound / chunk) + n_req    (fixed chunks, no work list)
 * A call with a work list of n_work segments needs
 * dspark_attn_workspace_bytes(n_work, 0, row_tiles, chunk) bytes.  Each
 * attention call is a chunk kernel plus a merge kernel on `stream`; calls
 * that share a workspace must not overlap in time.  Returns -1 on invalid
 * input.
 */
int64_t dspark_attn_workspace_bytes(int n_req, int64_t key_rows_bound, int row_tiles, int chunk);

/*
 * Work lists (int32, device memory, built by the caller; not validated on
 * the device beyond clamping the run ranges to [0, n_work]).
 *
 * varlen / verify: segment lists.  A segment is keys [k0, k1) of one
 * request.  Workgroup (run w, KV head g) processes the records of run w;
 * n_groups must be a multiple of 8, and the 8 workgroups of run w run on
 * XCD w mod 8 (so a plan can size each XCD's runs to its measured speed):
 *   [n_work][8] segment records, grouped by run:
 *       request, k0, k1, partial slot (-1 when the request has one segment,
 *       which then writes the output), first query row, query length,
 *       key length, first key row (varlen) or resident slot (verify)
 *   [n_groups + 1] run ranges: run w holds records range[w] .. range[w+1]
 *   [n_req][4] request records: first partial slot, segment count,
 *       first query row, query length
 * The segments of a request must cover its keys exactly once, and a split
 * request's segments must use consecutive partial slots in key order (the
 * merge folds them in slot order).  Cuts at the same key positions give
 * bit-identical outputs; a balanced plan (equal keys per run) moves the cuts
 * with the batch, a request-local plan (cuts at multiples of a fixed chunk)
 * makes every request's output independent of the batch.
 * Without a list (work == NULL) a persistent grid walks fixed chunks of
 * `chunk` keys in request order: the launch depends only on n_req,
 * key_rows_bound and max_q (the capacity-tail kernel relies on this).
 *
 * draft: segment lists of the same shape over the context rows each request
 * streams (0 .. its largest anchor): workgroup (run w, KV head g) processes
 * the records of run w:
 *   [n_work][8] segment records, grouped by run: request, k0, k1, partial
 *       slot (-1: one segment), first block, block count, largest anchor,
 *       0 or 1 + ctx_off[request] (when given, the kernel starts the
 *       context loads without reading ctx_off first)
 *   [n_groups + 1] run ranges
 *   [n_req][4] request records: first partial slot, segment count, first
 *       block, block count
 * The segment with k1 equal to the largest anchor (the last) also attends
 * the blocks' own rows.  Without a list, workgroup (chunk, KV head) runs a
 * fixed chunk of `chunk` context rows, chunks in request order.
 *
 * Packed varlen attention, bottom-right causal (causal=1) or noncausal.
 * q [q_rows,16,128], k/v [k_rows,8,128], cu_q/cu_k int32 [n_req+1].
 * Request r attends queries cu_q[r]..cu_q[r+1] to keys cu_k[r]..cu_k[r+1];
 * causal query i of a request with q queries and k keys sees keys j <= k-q+i.
 * Key rows beyond cu_k[n_req] (a capacity tail) are never read.
 * Replaces aten::_flash_attention_forward as called by
 *   dspark_qwen/rocm_varlen.py:111-114          (PinnedRocmVarlenKernel.__call__, causal)
 *   dspark_qwen/packed_draft.py:26-29           (PinnedRocmDraftKernel.__call__, noncausal)
 *   dspark_qwen/persistent_qwen_target.py:231-234 (_native_attention, capacity tail)
 */
int dspark_varlen_attn_fwd(const void* q, const void* k, const void* v,
                           const int32_t* cu_q, const int32_t* cu_k, int n_req,
                           int64_t q_rows, int64_t k_rows, int max_q, int causal,
                           float scale, int chunk, const int32_t* work, int n_work, int n_groups,
                           void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Fused verification attention over the persistent KV store.
 * k_res/v_res: one layer of the resident store; element (slot, head, pos, d)
 * at slot*slot_stride + head*head_stride + pos*tok_stride + d (elements;
 * head-major [slots, 8, cap, 128] is 8*cap*128, cap*128, 128).
 * k_scr/v_scr: the same layer of the scratch, [max_q, 8, 128].
 * cu_q/cu_k: int32 [n_req+1] as built by dspark_txn_metadata; slots: int32 [n_req].
 * Request r sees its committed context (resident rows slot*cap .. +c) followed
 * by its staged rows (scratch rows cu_q[r] ..), bottom-right causal.
 * Replaces the per-layer pair prepare_attention + kernel call:
 *   dspark_qwen/persistent_target_kv.py:441-460 (capacity gather, fused here)
 *   dspark_qwen/persistent_qwen_target.py:223-234 (_native_attention)
 * key_rows_bound >= cu_k[n_req] (the bucket key capacity) fixes the grid.
 */
int dspark_verify_attn_fwd(const void* q, const void* k_res, const void* v_res,
                           const void* k_scr, const void* v_scr,
                           const int32_t* cu_q, const int32_t* cu_k, const int32_t* slots,
                           int n_req, int64_t slot_stride, int64_t tok_stride, int64_t head_stride,
                           int64_t key_rows_bound, int max_q, float scale, int chunk,
                           const int32_t* work, int n_work, int n_groups, void* out,
                           void* workspace, int64_t workspace_bytes, void* stream);

/*
 * dspark_verify_attn_fwd without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * and harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The split-K partials live in a static device array of
 * dspark_noalloc_scratch_bytes() bytes (32 MiB) that each GPU holds until
 * the process ends; a call whose partials need more (see
 * dspark_attn_workspace_bytes) returns -1 and launches nothing.  The call
 * allocates nothing, and its result is bit-identical to
 * dspark_verify_attn_fwd's.  Every call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU (other streams, other threads) race.
 * The array's address is resolved on the first call on each device, which
 * must be the current device.
 */
int64_t dspark_noalloc_scratch_bytes(void);
int dspark_verify_attn_fwd_noalloc(const void* q, const void* k_res, const void* v_res,
                                   const void* k_scr, const void* v_scr,
                                   const int32_t* cu_q, const int32_t* cu_k, const int32_t* slots,
                                   int n_req, int64_t slot_stride, int64_t tok_stride, int64_t head_stride,
                                   int64_t key_rows_bound, int max_q, float scale, int chunk,
                                   const int32_t* work, int n_work, int n_groups, void* out, void* stream);

/*
 * dspark_verify_attn_fwd with the layer's staging fused in: the new rows are
 * read from k_new/v_new ([q_rows, 8, 128], the model's projected K/V) and
 * copied into k_scr/v_scr by the workgroups that read them, replacing the
 * separate dspark_kv_stage launch of stage_layer
 * (dspark_qwen/persistent_target_kv.py:427-438).  Scratch contents after the
 * call equal those after dspark_kv_stage; outputs are bit-identical to the
 * unfused pair.  k_new/v_new must not alias the scratch.
 */
int dspark_verify_attn_staged_fwd(const void* q, const void* k_res, const void* v_res,
                                  const void* k_new, const void* v_new, void* k_scr, void* v_scr,
                                  const int32_t* cu_q, const int32_t* cu_k, const int32_t* slots,
                                  int n_req, int64_t slot_stride, int64_t tok_stride, int64_t head_stride,
                                  int64_t key_rows_bound, int max_q, float scale, int chunk,
                                  const int32_t* work, int n_work, int n_groups, void* out,
                                  void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Multi-block DSpark draft attention.  Request r owns blocks
 * cu_blocks[r]..cu_blocks[r+1] (1..8 blocks), each 7 query rows; block b
 * sees context positions j < anchors[b] of its request plus its own 7 rows
 * (bidirectional), never another block.  Context row j of request r lives at
 *   k_ctx + phys*tok_stride + head*head_stride,
 *   phys = ctx_idx ? ctx_idx[ctx_off[r] + j] : ctx_off[r] + j,
 * so both a slotted pool ([slots*cap, 8, 128]) and the append-order pool of
 * dspark_qwen/packed_draft.py ([1, 8, N, 128] with gather indices) are read
 * in place.  Every ctx_idx entry a request addresses lies in [0, 2^31): the
 * kernel reads the low 32 bits.  q/out [7*n_blocks,16,128]; k_blk/v_blk [7*n_blocks,8,128].
 * V (context and block) and out are bf16.  q_dtype / k_dtype select bf16 (0)
 * or fp32 (1) for Q and for K (context and block K share one type, with the
 * same element strides as V): fp32 values are rounded to bf16 (nearest even)
 * as they are loaded, which is the autocast boundary cast of the reference's
 * AMP pool (FP32 K, BF16 V; packed_draft.py:222-235), so an fp32-K pool gives
 * the same output bits as a bf16 pool holding the rounded values.
 * Replaces the cat + index_select + cast + noncausal kernel sequence of
 *   dspark_qwen/packed_draft.py:219-236 (PackedDraft.backbone)
 * with the block_mask semantics of dspark_qwen/model.py:12-19.
 *
 * Scheduling: with workgroups = 0 the grid holds one workgroup per (run,
 * KV head) of the work list (or per fixed chunk without one).  With
 * workgroups > 0 (a multiple of 8; one per CU fills the chip) the grid is
 * that many persistent workgroups taking (run, KV head) items, runs in
 * list order, from ticket counters in `queue`: queues = 1 shares one queue,
 * queues = 8 gives each KV head its own queue served by workgroups
 * b = head (mod 8).  queue holds 2 int32 per queue, must be zero before the
 * first call and is zero again after every call (the last workgroup resets
 * it); calls sharing one queue buffer must not overlap.  The persistent
 * mode needs a work list of one segment per run (n_work == n_groups) and
 * seg_anchors: 8 int32 per segment record, the anchors of the record's
 * blocks b0 .. b0+nb-1 then any padding (16-byte aligned; NULL otherwise).
 * Outputs do not depend on the mode.
 */
int dspark_draft_attn_fwd(const void* q, int q_dtype, const void* k_ctx, const void* v_ctx,
                          int k_dtype, const int64_t* ctx_idx, const int64_t* ctx_off,
                          const int32_t* ctx_len, int64_t tok_stride, int64_t head_stride,
                          const void* k_blk, const void* v_blk,
                          const int32_t* cu_blocks, const int32_t* anchors,
                          int n_req, int64_t ctx_rows_bound, int max_blocks, float scale, int chunk,
                          const int32_t* work, int n_work, int n_groups,
                          int workgroups, int queues, int32_t* queue, const int32_t* seg_anchors,
                          void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Verify-layer prologue (the Qwen3 attention steps before the KV cache
 * update, as run by dspark_qwen/persistent_qwen_target.py:45-95 through
 * transformers' Qwen3Attention): for every token t of x [tokens, hidden]
 *   q = RoPE(RMSNorm(x Wq^T, q_norm)), k = RoPE(RMSNorm(x Wk^T, k_norm)), v = x Wv^T
 * per 128-dim head; W* in nn.Linear layout ([16*128 | 8*128, hidden]),
 * RMSNorm y = w x / sqrt(mean(x^2) + eps), RoPE rotate-half with angle
 * positions[t] * inv_freq[d] (float32 table of 64 entries).  rope
 * (optional, NULL forms the angles in the kernel): the rows' cos/sin table
 * written by dspark_rope_table for these positions and inv_freq - the same
 * bits, without the per-layer sincos.  q_out [tokens, 16, 128];
 * k_out/v_out token rows of 8*128 elements, kv_row_stride apart (1024
 * writes a [tokens, 8, 128] tensor, e.g. the transaction scratch layer,
 * replacing stage_layer's copy).  hidden must be a multiple of 128.  x, the
 * weights, outputs, inv_freq and rope 16-byte aligned, q_norm/k_norm 8-byte
 * aligned.  FP32 accumulation, bf16 outputs.
 */
int dspark_qkv_prologue(const void* x, const void* wq, const void* wk, const void* wv,
                        const void* q_norm, const void* k_norm, const float* inv_freq,
                        const int64_t* positions, const float* rope, int tokens, int hidden, float eps,
                        void* q_out, void* k_out, void* v_out, int64_t kv_row_stride, void* stream);

/*
 * Rotary table of a set of rows: table[t][d] = cos(positions[t] * inv_freq[d]),
 * table[t][64 + d] = sin(...), d < 64, the angle formed in FP32 (float32
 * [tokens][128]).  Computed once per verification transaction and shared by
 * the prologues of all layers, as the model computes its position
 * embeddings once per forward (transformers' Qwen3RotaryEmbedding, called by
 * Qwen3Model.forward; the reference keeps them in the model dtype, this
 * table in float32).
 */
int dspark_rope_table(const float* inv_freq, const int64_t* positions, int tokens, float* table, void* stream);

/*
 * Draft context K/V projection: what DSpark's draft does to newly committed
 * target features after its fc layer, for all `layers` draft layers in one
 * launch, written into the slotted draft pool.  For token t of x
 * [tokens, hidden] (the fc output, before the context norm):
 *   ctx = RMSNorm(x_t, w_c),  k_l = RoPE(RMSNorm(ctx Wk_l^T, k_norm_l)),
 *   v_l = ctx Wv_l^T                                 (per 128-dim KV head)
 * w: [layers][2][8*128][hidden] bf16, the k_proj then v_proj weights of each
 * layer with the context norm weight folded in (W diag(w_c)); k_norm
 * [layers][128]; eps_ctx / eps_k the two RMSNorm epsilons; RoPE rotate-half
 * at the token's absolute position with inv_freq (64 float32).  req: int32
 * [n_req][4] records (pool slot, first position, first token, token count),
 * ordered by first token, the first at token 0, covering every token once;
 * token t of record r lands at position first_position + (t - first_token)
 * of slot `slot` in every layer: element (slot, head, pos, d) of layer l at
 * k_pool/v_pool + l*layer_stride + slot*slot_stride + head*head_stride +
 * pos*128 + d.  The caller keeps every position within its pool.  flag
 * (optional): set to 1 when an output is not finite (never cleared).
 * Replaces dspark_qwen/model.py:141-146 (DSparkDraft.project_context_kv)
 * after its fc, and the projection + cat of
 *   dspark_qwen/packed_draft.py:147-158 (PackedDraft.append_committed).
 */
int dspark_draft_kv_project(const void* x, int tokens, int hidden, const void* w, const void* k_norm,
                            int layers, const float* inv_freq, const int32_t* req, int n_req,
                            float eps_ctx, float eps_k, void* k_pool, void* v_pool, int64_t layer_stride,
                            int64_t slot_stride, int64_t head_stride, int32_t* flag, void* stream);

/*
 * The same projection after a library GEMM, for large appends: y [tokens,
 * y_stride] holds x Wfold^T (columns [layer][K, V][head][128], the folded
 * weights of dspark_draft_kv_project as one [layers*2*1024, hidden]
 * matrix), FP32 (y_dtype 1: the GEMM's accumulator, so that every output is
 * rounded to bf16 once, as dspark_draft_kv_project rounds it) or bf16
 * (y_dtype 0: the reference's autocast rounding of k_proj / v_proj); this
 * applies the context-norm factor of x's rows, k_norm and RoPE on K, and
 * stores K/V into the pool exactly as dspark_draft_kv_project does.  Row i
 * of y and x is token token0 + i of the records, so a long append can be
 * projected in chunks.  Same flag convention.
 * Replaces the same reference code as dspark_draft_kv_project.
 */
int dspark_draft_kv_epilogue(const void* y, int y_dtype, int64_t y_stride, const void* x, int tokens, int token0,
                             int hidden, const void* k_norm, int layers, const float* inv_freq,
                             const int32_t* req, int n_req, float eps_ctx, float eps_k, void* k_pool,
                             void* v_pool, int64_t layer_stride, int64_t slot_stride, int64_t head_stride,
                             int32_t* flag, void* stream);

/*
 * Float64 sampling law and speculative verification (the consumer of the
 * verification round, after the LM head), following
 * dspark_qwen/tensor_sampling.py.  logits: [rows, >= vocab] bf16 (dtype 0)
 * or fp32 (dtype 1), row_stride elements apart.
 *
 * dspark_logit_row_stats: per row and chunk of 8192 logits, the max of
 * x / temperature and the sum of exp(x / temperature - max) (float64 pairs,
 * dspark_row_stats_bytes(rows, vocab) bytes); bad[row] is set to 1 when a
 * logit or its scaled value is not finite (the caller zeroes `bad` first).
 * Replaces the softmax of logits_to_probabilities (tensor_sampling.py:37-48)
 * for callers that never need the law materialised.
 */
int64_t dspark_row_stats_bytes(int rows, int vocab);
int dspark_logit_row_stats(const void* logits, int dtype, int rows, int vocab, int64_t row_stride,
                           double temperature, double* stats, int32_t* bad, void* stream);

/*
 * dspark_spec_verify: verify_proposal (tensor_sampling.py:114-162) for every
 * request at once.  Request r owns logit rows cu_rows[r] .. cu_rows[r+1]
 * (n_r + 1 rows), draft tokens / draft law rows cu_rows[r] - r .. + n_r of
 * tokens (int64) and q (float64 [.., vocab]), and draws its uniforms from
 * uniforms[cu_rows[r] ..] in the reference's order (at most n_r + 1).
 * budget[r] is the remaining output budget; stops the EOS ids.  Outputs:
 * the emitted tokens at out_tokens[cu_rows[r] ..] and out_meta[r][8] =
 * {emitted, accepted draft tokens, rejected index (-1 none), extra (0 none,
 * 1 residual, 2 bonus), stop (0 round complete, 1 eos, 2 budget), uniforms
 * used, error (0 ok, 1 token outside the vocabulary, 2 zero q at a proposed
 * token, 3 non-finite logits, 4 zero residual mass, 5 uniform outside
 * [0, 1), 6 more than 255 proposed tokens), 0}.  stats/bad from dspark_logit_row_stats with the same
 * temperature.  The q rows are read at the proposed tokens and, on a
 * rejection, in full; their sums are not checked.  Three launches: one lane
 * per request decides, then the final draws (see below).  workspace:
 * dspark_draw_workspace_bytes(n_req) bytes, 64-byte aligned.
 *
 * Categorical draws (the final draw of a verification, and
 * dspark_sample_rows): the first index whose running sum of the law exceeds
 * u, else the last index of positive mass (sample_categorical,
 * tensor_sampling.py:69-76), computed as 256 segment sums per draw, a scan,
 * and a walk of one segment.
 */
int64_t dspark_draw_workspace_bytes(int jobs);
int dspark_spec_verify(const void* logits, int dtype, int64_t row_stride, int vocab, double temperature,
                       const double* stats, const int32_t* bad, const int32_t* cu_rows, int n_req,
                       const int64_t* tokens, const double* q, const double* uniforms,
                       const int32_t* budget, const int32_t* stops, int n_stops, int64_t* out_tokens,
                       int32_t* out_meta, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * dspark_logits_to_probs: the float64 law rows probs [rows, vocab] from the
 * logits and their row statistics (logits_to_probabilities,
 * tensor_sampling.py:37-48).  dspark_sample_rows: one categorical draw per
 * row of float64 laws probs [rows, vocab] with uniforms[row] in [0, 1)
 * (sample_categorical, tensor_sampling.py:69-76); workspace
 * dspark_draw_workspace_bytes(rows) bytes, 64-byte aligned.
 */
int dspark_logits_to_probs(const void* logits, int dtype, int rows, int vocab, int64_t row_stride,
                           double temperature, const double* stats, double* probs, void* stream);
int dspark_sample_rows(const double* probs, int rows, int vocab, const double* uniforms, int64_t* out,
                       void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Transaction metadata of PersistentTargetKV.begin
 * (dspark_qwen/persistent_target_kv.py:392-411), built on the device from
 * req = int32 [3][n_req] (slot, committed context, query length per request):
 * committed_idx/scratch_idx int64 [key_capacity], from_scratch/valid
 * uint8 [key_capacity], positions int64 [query_tokens], cu_q/cu_k int32
 * [n_req+1].  Bit-exact with the reference lists, capacity tail included.
 */
int dspark_txn_metadata(const int32_t* req, int n_req, int64_t ctx_capacity,
                        int64_t key_capacity, int64_t query_tokens,
                        int64_t* committed_idx, int64_t* scratch_idx,
                        uint8_t* from_scratch, uint8_t* valid, int64_t* positions,
                        int32_t* cu_q, int32_t* cu_k, void* stream);

/*
 * Stage one layer's new K/V rows into scratch
 * (dspark_qwen/persistent_target_kv.py:436-437, stage_layer).
 */
int dspark_kv_stage(const void* k_new, const void* v_new, void* k_scr_layer, void* v_scr_layer,
                    int64_t rows, int64_t row_bytes, void* stream);

/*
 * Commit the accepted prefix n_accepted[r] of every request for all layers
 * in one launch: scratch rows cu_q[r]..+n -> resident positions c..c+n of
 * the request's slot (dspark_qwen/persistent_target_kv.py:479-483).  Rows
 * n..q-1 are rolled back by omission.  req as for dspark_txn_metadata
 * (pre-commit context).  Resident piece (layer, slot, head, pos) of
 * piece_bytes starts at layer*layer_stride + slot*slot_stride +
 * head*head_stride + pos*tok_stride (bytes); scratch is [L, scratch_rows,
 * heads * piece_bytes].
 */
int dspark_kv_commit(void* k_res, void* v_res, const void* k_scr, const void* v_scr,
                     const int32_t* req, const int32_t* cu_q, const int32_t* n_accepted,
                     int n_req, int max_q, int layers, int64_t layer_stride, int64_t slot_stride,
                     int64_t head_stride, int64_t tok_stride, int64_t ctx_capacity, int heads,
                     int64_t piece_bytes, int64_t scratch_rows, void* stream);

/*
 * Materialised capacity-length K/V of prepare_attention
 * (dspark_qwen/persistent_target_kv.py:452-459), token-major out:
 * row j = valid[j] ? (from_scratch[j] ? scratch[scratch_idx[j]]
 *                                     : resident(slot, pos) with committed_idx[j] = slot*cap+pos) : 0.
 * Resident geometry (bytes) as for dspark_kv_commit, one layer.
 */
int dspark_kv_gather(const void* k_res_layer, const void* v_res_layer,
                     const void* k_scr_layer, const void* v_scr_layer,
                     const int64_t* committed_idx, const int64_t* scratch_idx,
                     const uint8_t* from_scratch, const uint8_t* valid,
                     int64_t key_capacity, int64_t slots, int64_t slot_stride, int64_t head_stride,
                     int64_t tok_stride, int64_t ctx_capacity, int heads, int64_t piece_bytes,
                     int64_t scr_rows, void* k_out, void* v_out, void* stream);

/*
 * Packed varlen layout of PackedLayout.from_metadata
 * (dspark_qwen/varlen_target.py:28-60), built on the device.
 * Inputs: int64 query markers/positions [nq] and key markers/positions [nk].
 * Requests are the runs of equal consecutive query markers (at most max_req,
 * max_req <= 8192).  Outputs: cu_q/cu_k int32 [max_req+1] (first B+1 used),
 * gather int64 [nk] (first sum-K used: every request's keys in physical
 * order, requests in query order), and summary int64 [4 + 3*max_req]:
 *   [0] 0 ok | 1 a request's queries are not one contiguous run |
 *       2 keys are not the complete prefix 0..k-1 (or k < q) |
 *       3 query positions are not k-q..k-1 | 4 more than max_req requests
 *   [1] first failing request (query order; prefix checked before suffix)
 *   [2] B, [3] sum K, [4+r] marker, [4+max_req+r] q_r, [4+2*max_req+r] k_r.
 * The caller reads the summary once (the reference also synchronises) and
 * raises the reference's ValueError for codes 1-3.
 */
int64_t dspark_layout_workspace_bytes(int64_t nq, int64_t nk, int max_req);
int dspark_layout_build(const int64_t* query_requests, const int64_t* query_positions, int64_t nq,
                        const int64_t* key_requests, const int64_t* key_positions, int64_t nk,
                        int max_req, int32_t* cu_q, int32_t* cu_k, int64_t* gather,
                        int64_t* summary, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * PackedLayout.gather_kv (dspark_qwen/varlen_target.py:74-82): rows
 * indices[0..n_rows) of a [heads, src_rows, piece] pool layer (byte strides
 * head_stride, row_stride) into token-major [n_rows, heads, piece] outputs,
 * K and V in one launch.  Indices outside [0, src_rows) produce zero rows.
 */
int dspark_pool_gather(const void* k_src, const void* v_src, int64_t src_rows, int64_t head_stride,
                       int64_t row_stride, int heads, int64_t piece_bytes, const int64_t* indices,
                       int64_t n_rows, void* k_dst, void* v_dst, void* stream);

/*
 * Draft context pool append (dspark_qwen/packed_draft.py:130-168
 * append_committed: the cat of projected K/V onto the pool).  The pool is
 * one tensor per K and V, [layers, slots, heads, capacity, piece] or any
 * order expressed by the byte strides (as for dspark_kv_commit).  Per layer
 * l, k_src[l]/v_src[l] (a host array of device pointers, layers <= 16) hold
 * the new rows of all requests in chunk order, row i of head h at
 * h*src_head_stride + i*src_row_stride bytes.  req = int32 [4][n_req]:
 * slot, first position, first source row (ascending), row count.  Rows are
 * written beyond the caller's committed lengths, so the append becomes
 * visible only when the caller advances them.  nonfinite (optional, int32)
 * is set to 1 if any appended element is Inf/NaN (elem_bytes 2 = bf16,
 * 4 = fp32).  Either pool may be NULL (with its source array) to append K
 * or V alone, e.g. the two halves of a pool whose K and V types differ.
 */
int dspark_pool_append(void* k_pool, void* v_pool, int64_t layer_stride, int64_t slot_stride,
                       int64_t head_stride, int64_t tok_stride, int64_t capacity, int heads,
                       int64_t piece_bytes, int elem_bytes, int layers,
                       const void* const* k_src, const void* const* v_src,
                       int64_t src_head_stride, int64_t src_row_stride, int64_t src_rows,
                       const int32_t* req, int n_req, int32_t* nonfinite, void* stream);

/*
 * Append-order KV cache of PackedTarget (dspark_qwen/packed_target.py:30-113):
 * per layer K/V [1, H, N, piece] with rows in append order and int64
 * key_requests / key_positions [N].
 *
 * dspark_crop_plan: the keep mask of crop (packed_target.py:99-108),
 * keep = (request != marker) | (position < length), as a stable compaction:
 * plan[j] = source row of kept row j, and the compacted markers/positions.
 * The caller knows the kept count (N minus the cropped rows).
 * Workspace: dspark_crop_plan_workspace_bytes(N).
 */
int64_t dspark_crop_plan_workspace_bytes(int64_t n);
int dspark_crop_plan(const int64_t* key_requests, const int64_t* key_positions, int64_t n,
                     int64_t marker, int64_t length, int64_t* plan, int64_t* out_requests,
                     int64_t* out_positions, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Rebuild `tensors` (<= 64) row tensors [H, rows, piece] in one launch
 * (src/add/dst: host arrays of device pointers).  With plan: output row j =
 * src row plan[j] (crop / gather, n_out <= n_old).  Without: output rows are
 * the n_old src rows then the n_add add rows (append: the reference's
 * torch.cat along the row axis, packed_target.py:159-168 and
 * packed_draft.py:159-161).
 */
int dspark_rows_rebuild(const void* const* src, const void* const* add, void* const* dst, int tensors,
                        int heads, int64_t piece_bytes, int64_t n_old, int64_t n_add,
                        const int64_t* plan, int64_t n_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSPARK_AMD_H */
