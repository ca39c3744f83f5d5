/*
 * wkv7.h -- C ABI of the MI355X (gfx950) WKV7 slot-pool library, libwkv7.so.
 *
 * The reference (xiaol/wkvm) is pure Python: it keeps request state in a
 * layer-major slot pool (wkvm/runner/state.py:35-46) and runs the WKV7
 * recurrence through the third-party `fla` package's Triton kernels
 * (wkvm/models/rwkv7.py:108-113) between gather/scatter copies of the pool.
 * Each entry point below replaces one of those operations; the comment on each
 * names the reference code it stands in for. The Python host package
 * `wkvm_amd` binds these symbols with ctypes (wkvm_amd/_lib.py lists every
 * signature).
 *
 * Conventions (all entry points):
 *  - Memory: every pointer is caller-owned device memory (except where a
 *    parameter says "host"). The library never allocates, frees or
 *    synchronises; work is enqueued on `stream` (a hipStream_t, or NULL for
 *    the default stream) and is asynchronous to the host.
 *  - Slot pool layout (wkvm/runner/state.py:35-46): one layer of the wkv
 *    family is a contiguous fp32 tensor [num_rows, H, 64, 64] with
 *    num_rows = num_slots + 1 (row 0 is the reserved pad slot,
 *    wkvm/core/arena.py:32-37). Element [row, h, j, i] is the state entry for
 *    key index j and value index i (h = S^T of S_t = S_{t-1} diag(w) + ...).
 *  - Per-token vectors r, w, k, v, a, b are bf16 (passed as uint16_t bit
 *    patterns), contiguous [tokens, H, 64]. `w` is LOG-decay: the
 *    multiplicative decay applied to the state is exp(w), computed in fp32.
 *    This is the convention of the fla wkv op the reference calls.
 *  - Recurrence, per token and head (fp32 arithmetic):
 *        p_i     = sum_j a[j] h[j][i]
 *        h[j][i] = exp(w[j]) h[j][i] + b[j] p_i + k[j] v[i]
 *        y[i]    = sum_j (scale r[j]) h[j][i]
 *  - Slot ids are int32 in device memory. A kernel never touches memory
 *    outside [0, num_rows): rows whose id is out of range are skipped (the
 *    decode entry points write zeros into such a row's outputs). Host
 *    wrappers validate ids before launch and raise instead.
 *  - Return value: 0 on success, a negative WKV7_ERR_* code for rejected
 *    arguments (nothing is enqueued), or a positive hipError_t from the launch.
 *  - Thread safety: calls are stream-ordered; two calls that write the same
 *    slot rows on different streams race.
 */
#ifndef WKV7_H
#define WKV7_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WKV7_ABI_VERSION 10

#define WKV7_OK 0
#define WKV7_ERR_ARG (-1)       /* null pointer, negative size, bad enum */
#define WKV7_ERR_SHAPE (-2)     /* row size beyond the slot stride, misaligned inputs */
#define WKV7_ERR_WORKSPACE (-3) /* workspace missing or too small */

#define WKV7_Y_BF16 0 /* y written as bf16 (round to nearest even) */
#define WKV7_Y_F32 1  /* y written as fp32 */

#define WKV7_TO_HOST 0   /* wkv7_slot_transfer: device slot rows -> host */
#define WKV7_FROM_HOST 1 /* wkv7_slot_transfer: host -> device slot rows */

/* ABI version of the loaded library (WKV7_ABI_VERSION at build time). */
int wkv7_abi_version(void);

/* Human-readable text for a return code (WKV7_ERR_* or hipError_t). */
const char *wkv7_strerror(int code);

/*
 * One decode step (one token per slot) for B slots of one layer, in place.
 *
 * Replaces, per layer of RWKV7Runner.decode_step (wkvm/runner/runner.py:65-89):
 * the `index_select` gather of the batch's wkv rows
 * (wkvm/runner/state.py:77), fla's fused recurrent WKV7 kernel on the gathered
 * [B, H, K, V] state (dispatched for seq_len < 64, wkvm/models/rwkv7.py:110-111),
 * and the `index_copy_` scatter back (wkvm/runner/state.py:91). State is read
 * and written at its slot row; nothing is gathered.
 *
 *   wkv_layer  [num_rows, H, 64, 64] fp32, updated in place at rows slot_ids[b]
 *   slot_ids   [B] int32 (device); must be distinct (duplicates race)
 *   row_order  [B] int32 (device) or NULL: the order in which batch rows are
 *              visited, a permutation of 0..B-1. Results do not depend on it;
 *              rows sorted by slot id keep the HBM stream inside a few
 *              neighbouring slot regions and raise bandwidth when slots are
 *              scattered through the pool. Entries outside [0, B) are skipped.
 *   r..b       [B, H, 64] bf16
 *   y          [B, H, 64], dtype per y_dtype (WKV7_Y_BF16 | WKV7_Y_F32); a
 *              row whose slot id is outside [0, num_rows) gets y = 0 and its
 *              state is not touched
 */
int wkv7_decode_slots(float *wkv_layer, int64_t num_rows, int32_t H,
                      const int32_t *slot_ids, const int32_t *row_order, int32_t B,
                      const uint16_t *r, const uint16_t *w, const uint16_t *k,
                      const uint16_t *v, const uint16_t *a, const uint16_t *b,
                      void *y, int32_t y_dtype, float scale, void *stream);

/*
 * One decode step (one token per row) with the state read from one tensor and
 * written to another: row b reads state_in[in_ids[b]] and writes
 * state_out[out_ids[b]] (both [rows, H, 64, 64] fp32). The arithmetic is
 * wkv7_decode_slots'; with state_in == state_out and in_ids == out_ids it is
 * that call.
 *
 * Replaces fla's recurrent WKV7 op at seq_len 1 as the reference's model
 * layer calls it (dispatched for seq_len < 64, wkvm/models/rwkv7.py:108-111;
 * reached from RWKV7Runner.decode_step, wkvm/runner/runner.py:74-76):
 * fused_recurrent_rwkv7(r, w, k, v, a, b, initial_state=, output_final_state=)
 * reads initial_state and returns a new final_state tensor.
 *
 *   state_in   NULL = zero initial state (fla's initial_state=None)
 *   in_ids     [B] int32 (device), or NULL: row b reads state row b
 *   state_out  NULL = the new state is not written (output_final_state=False)
 *   out_ids    [B] int32 (device), or NULL: row b writes state row b; must be
 *              distinct, and no row may write a state row another row reads
 *   in_rows, out_rows   rows of each tensor (at least B where its ids are NULL,
 *              else WKV7_ERR_SHAPE); ids outside [0, rows) give y = 0 and no
 *              state write for that row
 *   H, row_order, B, r..b, y, y_dtype, scale   as wkv7_decode_slots
 * Ids without their tensor are WKV7_ERR_ARG.
 */
int wkv7_decode_into(const float *state_in, int64_t in_rows, const int32_t *in_ids,
                     float *state_out, int64_t out_rows, const int32_t *out_ids,
                     int32_t H, const int32_t *row_order, int32_t B,
                     const uint16_t *r, const uint16_t *w, const uint16_t *k,
                     const uint16_t *v, const uint16_t *a, const uint16_t *b,
                     void *y, int32_t y_dtype, float scale, void *stream);

/*
 * Chunked prefill of nseq ragged sequences of one layer; each sequence starts
 * from its slot's state (or from zero when zero_init != 0) and leaves its
 * final state in that slot.
 *
 * Replaces, per layer, fla's `chunk_rwkv7` (chunk 64) and its fused recurrent
 * tail as called by RWKV7Runner.prefill (wkvm/runner/runner.py:41-63, one
 * request per call from Engine._execute, wkvm/engine.py:152-155), together
 * with the per-chunk gather/scatter round trip through the bank
 * (wkvm/runner/state.py:63-97). Ragged batching follows the cu_seqlens
 * (q_start_loc) contract of MixedBatchMetadata (wkvm/core/mixed_batch.py:213-270).
 *
 *   wkv_layer     [num_rows, H, 64, 64] fp32
 *   slot_ids      [nseq] int32 (device), distinct
 *   cu_seqlens    [nseq + 1] int32 (device), cu_seqlens[0] = 0,
 *                 non-decreasing, cu_seqlens[nseq] = total_tokens
 *   seq_order     [nseq] int32 (device) or NULL: the order in which the
 *                 sequences are started (a permutation of 0..nseq-1; NULL =
 *                 0..nseq-1). Longest first packs ragged batches onto the
 *                 compute units with the least idle tail; results do not
 *                 depend on it
 *   r..b          [total_tokens, H, 64] bf16, 16-byte aligned (else WKV7_ERR_SHAPE)
 *   y             [total_tokens, H, 64], dtype per y_dtype; 8-byte aligned for
 *                 bf16, 16-byte for fp32 (whole rows are stored as vectors;
 *                 else WKV7_ERR_SHAPE); a sequence whose slot id is outside
 *                 [0, num_rows) gets y = 0 and its state is not touched
 *
 * Decay range: the chunked form scales operands by exp(+-G) with G a sum of
 * up to 16 consecutive log-decays, so every w must be >= -5 (exp(80) is
 * within fp32 and bf16 range; RWKV-7's w lies in (-0.61, 0]). Stronger
 * decays overflow to inf/NaN; the decode step has no such limit.
 */
int wkv7_prefill_varlen(float *wkv_layer, int64_t num_rows, int32_t H,
                        const int32_t *slot_ids, const int32_t *cu_seqlens,
                        const int32_t *seq_order, int32_t nseq, int64_t total_tokens,
                        const uint16_t *r, const uint16_t *w, const uint16_t *k,
                        const uint16_t *v, const uint16_t *a, const uint16_t *b,
                        void *y, int32_t y_dtype, int32_t zero_init, float scale,
                        void *stream);

/* Run flags of wkv7_prefill_runs. */
#define WKV7_RUN_INIT_ZERO 1      /* start from zero state */
#define WKV7_RUN_INIT_IDENTITY 2  /* start from the identity (takes precedence) */
#define WKV7_RUN_KV_ZERO 4        /* read k and v as zero */
#define WKV7_RUN_Y_ALT 8          /* write y to y_alt */
#define WKV7_RUN_STATE_ALT 16     /* slot_ids[run] is a row of state_alt, not of wkv_layer */

/*
 * wkv7_prefill_varlen over "runs" with per-run options, for the segmented
 * prefill of few long sequences (with wkv7_segment_chain and
 * wkv7_segment_correct below). It has no single counterpart in the reference:
 * together the three compute what one chunk_rwkv7 call of RWKV7Runner.prefill
 * computes (wkvm/runner/runner.py:41-63, wkvm/models/rwkv7.py:108-113), with
 * the sequence's segments running side by side.
 *
 * Runs [0, n_primary) take their token ranges from cu_seqlens (as
 * wkv7_prefill_varlen, n_primary + 1 entries); run n_primary + i takes tokens
 * [cu_alt[2i], cu_alt[2i+1]) of the same inputs. run_flags [nseq] (device,
 * WKV7_RUN_* bits, NULL = all 0) select the initial state, zero k and v, and
 * redirect y to y_alt (same shape, dtype and alignment as y) and the state to
 * state_alt [alt_rows, H, 64, 64] fp32. A run's rows must be distinct from
 * every other run's. With state_in [in_rows, H, 64, 64] fp32 (NULL = none),
 * a run that starts from a stored state (no zero or identity flag, zero_init
 * 0) reads it from state_in row in_ids[run] (in_ids NULL: row `run`, which
 * needs in_rows >= nseq) instead of its slot row; its final state still goes
 * to the slot row. Rejected rows give y = 0 as in wkv7_prefill_varlen.
 */
int wkv7_prefill_runs(float *wkv_layer, int64_t num_rows, int32_t H,
                      const int32_t *slot_ids, const int32_t *cu_seqlens,
                      const int32_t *seq_order, int32_t nseq, int64_t total_tokens,
                      const uint16_t *r, const uint16_t *w, const uint16_t *k,
                      const uint16_t *v, const uint16_t *a, const uint16_t *b,
                      void *y, int32_t y_dtype, int32_t zero_init, float scale,
                      const int32_t *run_flags, const int32_t *cu_alt, int32_t n_primary,
                      float *state_alt, int64_t alt_rows, void *y_alt,
                      const float *state_in, int64_t in_rows, const int32_t *in_ids,
                      void *stream);

/*
 * Chunked prefill with the state read from one tensor and written to another:
 * sequence s reads its initial state from state_in[in_ids[s]] and writes its
 * final state to state_out[out_ids[s]] (both [rows, H, 64, 64] fp32). The
 * arithmetic is wkv7_prefill_varlen's; with state_in == state_out and
 * in_ids == out_ids it is that call.
 *
 * Replaces fla's chunk_rwkv7 as the reference's model layer calls it for
 * every prefill chunk (seq_len >= 64, wkvm/models/rwkv7.py:108-113; reached
 * from RWKV7Runner.prefill, wkvm/runner/runner.py:52-61):
 * chunk_rwkv7(r, w, k, v, a, b, initial_state=, output_final_state=,
 * cu_seqlens=) reads initial_state and returns a new final_state tensor, so
 * no copy of the state is needed.
 *
 *   state_in   NULL = zero initial state (fla's initial_state=None)
 *   in_ids     [nseq] int32 (device), or NULL: sequence s reads row s
 *   state_out  NULL = no final state written (output_final_state=False)
 *   out_ids    [nseq] int32 (device), or NULL: sequence s writes row s; must
 *              be distinct, and no sequence may write a state row another
 *              sequence reads
 *   in_rows, out_rows   rows of each tensor (at least nseq where its ids are
 *              NULL, else WKV7_ERR_SHAPE); a sequence with an id outside
 *              [0, rows) gets y = 0 and no state write
 *   H, cu_seqlens, seq_order, nseq, total_tokens, r..b, y, y_dtype, scale
 *              as wkv7_prefill_varlen (same alignment rules and decay range)
 * Ids without their tensor are WKV7_ERR_ARG.
 */
int wkv7_prefill_into(const float *state_in, int64_t in_rows, const int32_t *in_ids,
                      float *state_out, int64_t out_rows, const int32_t *out_ids, int32_t H,
                      const int32_t *cu_seqlens, const int32_t *seq_order, int32_t nseq,
                      int64_t total_tokens, const uint16_t *r, const uint16_t *w,
                      const uint16_t *k, const uint16_t *v, const uint16_t *a,
                      const uint16_t *b, void *y, int32_t y_dtype, float scale, void *stream);

/*
 * The state chain of a segmented prefill, per (sequence, head), in segment
 * order: hin[seg] = H_in, then H_in <- state_alt[main] + state_alt[phi] H_in.
 * H_in starts at wkv_layer[slot] (the state after segment 0) and ends there.
 *   seq_tab  [nseq][3] int32 (device): slot, first segment, segment count
 *   seg_tab  [nsegs][2] int32 (device): state_alt rows of the segment's zero-
 *            state run (H0) and of its identity run (Phi)
 *   hin      [nsegs, H, 64, 64] fp32 out: the state entering each segment
 */
int wkv7_segment_chain(float *wkv_layer, int64_t num_rows, int32_t H, const float *state_alt,
                       int64_t alt_rows, const int32_t *seq_tab, int32_t nseq,
                       const int32_t *seg_tab, int32_t nsegs, float *hin, void *stream);

/*
 * The output of a segmented prefill: for every token block,
 * y = y0 + q hin[seg] (seg >= 0) or y = y0 (seg < 0), per head, written in
 * y_dtype.
 *   y0, q    [total_tokens, H, 64] fp32 (the runs' y and y_alt)
 *   blk_tab  [nblk][3] int32 (device): first token, count (<= 64), segment
 */
int wkv7_segment_correct(int64_t total_tokens, int32_t H, const float *y0, const float *q,
                         const int32_t *blk_tab, int32_t nblk, const float *hin, int32_t nsegs,
                         void *y, int32_t y_dtype, void *stream);

/*
 * Copy slot rows between two slot-indexed tensors (or within one), bit-exact.
 *
 * A tensor here is `outer` blocks of `rows` slot rows; each slot row is
 * `row_bytes` contiguous bytes. Pair p copies, for every outer block o,
 *     src + o*src_outer_stride + src_ids[p]*src_slot_stride   (row_bytes)
 *  -> dst + o*dst_outer_stride + dst_ids[p]*dst_slot_stride.
 * A NULL id array means the identity (ids 0..n-1). Strides are in bytes.
 *
 * Replaces: the snapshot/restore slot-view copies of StateStore.save/load
 * (`bank.wkv[:, slot]`, `bank.shift[:, :, slot]`, wkvm/store.py:130-131 and
 * 151-152) as a device-to-device fork; the O(MB) copy StateArena.fork leaves
 * to the runner (wkvm/core/arena.py:82-93); and the per-layer
 * `index_select` / `index_copy_` of RWKV7StateBank.gather_cache /
 * scatter_cache (wkvm/runner/state.py:63-97), for which src (gather) or dst
 * (scatter) is a dense staging tensor with NULL ids.
 * Precondition: no dst row is written twice and no dst row is also a src row
 * (sources are not snapshotted first); duplicate src ids are allowed.
 */
int wkv7_slot_copy(void *dst, int64_t dst_outer_stride, int64_t dst_slot_stride,
                   int64_t dst_rows, const int32_t *dst_ids,
                   const void *src, int64_t src_outer_stride, int64_t src_slot_stride,
                   int64_t src_rows, const int32_t *src_ids,
                   int64_t outer, int64_t row_bytes, int32_t n, void *stream);

/*
 * Zero slot rows (admission reset: zero state == empty prefix).
 * Replaces RWKV7StateBank.zero_slots (wkvm/runner/state.py:50-54). Uses a fill
 * kernel, not a memset node, so it is safe inside captured HIP graphs.
 */
int wkv7_slot_zero(void *base, int64_t outer_stride, int64_t slot_stride, int64_t rows,
                   const int32_t *ids, int64_t outer, int64_t row_bytes, int32_t n,
                   void *stream);

/*
 * Copy one slot's rows of a slot-pool family between device memory and a
 * dense host buffer:
 *     host + o*row_bytes  <->  base + o*outer_stride + slot*slot_stride
 * for every outer block o < outer (`row_bytes` each; strides in bytes).
 * With staging == NULL the copy is one strided DMA (no kernel). With a
 * device staging buffer of at least outer*row_bytes bytes, the slot's rows
 * are gathered into (or scattered from) it by the copy kernel and the host
 * side moves as one contiguous DMA; strided device-to-host DMA runs at half
 * the host link's rate on some MI355X boxes, the contiguous one does not.
 * A staging buffer smaller than outer*row_bytes is WKV7_ERR_WORKSPACE.
 * direction: WKV7_TO_HOST or WKV7_FROM_HOST. `host` is a host pointer and
 * must be pinned (hipHostMalloc, torch pin_memory) for the copy to be
 * asynchronous; it holds the slot's rows densely, [outer][row_bytes], which
 * is the layout of the reference's WARM tensors (`bank.wkv[:, slot]` is
 * [L, H, K, V], `bank.shift[:, :, slot]` is [L, 2, D]).
 * Replaces the HOT <-> WARM copies of StateStore.save (wkvm/store.py:128-131,
 * D2H of bank.wkv[:, slot] and bank.shift[:, :, slot] into pinned host
 * tensors) and StateStore.load (wkvm/store.py:151-152, H2D into the slot
 * views). Returns WKV7_ERR_ARG for a slot outside [0, rows) or a bad
 * direction, WKV7_ERR_SHAPE if row_bytes exceeds a stride.
 */
int wkv7_slot_transfer(int32_t direction, void *host, void *base, int64_t outer_stride,
                       int64_t slot_stride, int64_t rows, int32_t slot, int64_t outer,
                       int64_t row_bytes, void *staging, size_t staging_bytes, void *stream);

/*
 * Token shift of one state family, fused with the lerp mixes that consume it,
 * for nseq ragged sequences (decode is nseq sequences of one token).
 *
 * For token t of sequence s (tokens cu_seqlens[s] .. cu_seqlens[s+1]-1):
 *     prev     = x[t-1], or the slot's cached row shift_rows[slot_ids[s]]
 *                for the sequence's first token
 *     delta    = bf16(prev - x[t])
 *     out[m,t] = bf16(fma(delta, mix[m], x[t]))    m = 0 .. n_mix-1
 * and the sequence's last row of x becomes the slot's cached row (in place).
 * A zero cached row is the zero shift-in at position 0 of a fresh sequence.
 *
 * Replaces the token-shift caches of the reference's RWKV-7 layers: the
 * attention mixer's conv_state and the channel mixer's ffn_state, held per
 * slot in bank.shift[:, 0] and bank.shift[:, 1] ([L, 2, S+1, D], model dtype,
 * wkvm/runner/state.py:40-46; semantics wkvm/models/rwkv7.py:17-27), which
 * the runner gathers into fla's Cache before each forward and scatters back
 * after it (wkvm/runner/state.py:78-79, 92-97). The shift and the
 * x + delta * mu mixes themselves run inside fla's RWKV7Attention /
 * RWKV7FeedForward (external, not in the reference).
 *
 *   x            [total_tokens, D] bf16, the mixer's input
 *   shift_rows   one layer and family of bank.shift: num_rows rows of D bf16,
 *                row_stride elements apart (bank.shift[l, f] has row_stride D)
 *   slot_ids     [nseq] int32 (device), distinct
 *   cu_seqlens   [nseq + 1] int32 (device), as for wkv7_prefill_varlen; NULL
 *                for a decode batch (sequence t is token t: nseq must equal
 *                total_tokens, else WKV7_ERR_ARG), which spares every token
 *                one dependent read before its slot id
 *   mix          [n_mix, D] bf16 (x_r, x_w, x_k, x_v, x_a, x_g for the
 *                attention mixer; x_k for the channel mixer)
 *   out          n_mix outputs of [total_tokens, D] bf16, out_stride elements
 *                apart
 * D, row_stride and out_stride must be multiples of 8 and x, shift_rows, mix
 * and out 16-byte aligned (else WKV7_ERR_SHAPE).
 */
int wkv7_token_shift_mix(const uint16_t *x, int64_t total_tokens, int32_t D,
                         uint16_t *shift_rows, int64_t num_rows, int64_t row_stride,
                         const int32_t *slot_ids, const int32_t *cu_seqlens, int32_t nseq,
                         const uint16_t *mix, int32_t n_mix, uint16_t *out,
                         int64_t out_stride, void *stream);

/*
 * RWKV-7 time-mix projections -> the WKV7 op's inputs, per token and head
 * (fp32 arithmetic, one bf16 rounding per output):
 *     a     = sigmoid(a_lora)                 w_out = -exp(-0.5) * sigmoid(w_lora)
 *     kk    = normalize(k * k_k) over the head (x / max(||x||_2, 1e-12))
 *     k_out = k * (1 + (a - 1) * k_a)         a_out = -kk      b_out = kk * a
 *     v_out = v + (v_first - v) * sigmoid(v_lora)   (v when v_lora is NULL)
 * w_lora, a_lora and v_lora are the LoRA outputs including their biases
 * (w0, a0, v0). w_out is the log-decay wkv7_decode_slots / _prefill_varlen
 * take.
 *
 * Replaces the element-wise part of fla's RWKV7Attention between its
 * projections and the wkv call (external; the reference calls it through the
 * model forward, wkvm/runner/runner.py:80-88, wkvm/models/rwkv7.py:108-113).
 *
 *   k, v, w_lora, a_lora, v_lora, v_first, outputs   [total_tokens, H*64] bf16
 *   k_k, k_a                                          [H*64] bf16
 * v_lora and v_first are both NULL (first layer) or both set. Pointers must
 * be 8-byte aligned (else WKV7_ERR_SHAPE).
 */
int wkv7_time_mix_inputs(int64_t total_tokens, int32_t H, const uint16_t *k,
                         const uint16_t *v, const uint16_t *w_lora, const uint16_t *a_lora,
                         const uint16_t *v_lora, const uint16_t *v_first,
                         const uint16_t *k_k, const uint16_t *k_a, uint16_t *w_out,
                         uint16_t *k_out, uint16_t *v_out, uint16_t *a_out, uint16_t *b_out,
                         void *stream);

/*
 * RWKV-7 time-mix output stage, per token and head (fp32 arithmetic, one
 * bf16 rounding per output):
 *     n   = (y - mean(y)) / sqrt(var(y) + eps) * ln_w + ln_b   (biased var)
 *     out = (n + (sum_c r k r_k) * v) * g
 * i.e. the per-head GroupNorm of the WKV output, the bonus term and the gate;
 * `out` is the input of the output projection.
 *
 * Replaces fla's g_norm, bonus and gate in RWKV7Attention (external; reached
 * through the model forward, wkvm/runner/runner.py:80-88).
 *
 *   y            [total_tokens, H, 64], dtype per y_dtype (the WKV output)
 *   r, k, v, g   [total_tokens, H*64] bf16 (k and v as fed to the WKV op)
 *   r_k          [H*64] bf16;  ln_w, ln_b [H*64] bf16 (GroupNorm affine)
 *   out          [total_tokens, H*64] bf16
 * Pointers must be 8-byte aligned, y 16-byte aligned when fp32 (else
 * WKV7_ERR_SHAPE).
 */
int wkv7_time_mix_output(int64_t total_tokens, int32_t H, const void *y, int32_t y_dtype,
                         const uint16_t *r, const uint16_t *k, const uint16_t *v,
                         const uint16_t *g, const uint16_t *r_k, const uint16_t *ln_w,
                         const uint16_t *ln_b, float eps, uint16_t *out, void *stream);

/*
 * The RWKV-7 time-mix decode of one token per slot, fused: for each batch
 * row and head,
 *     wkv7_time_mix_inputs -> wkv7_decode_slots (bf16 y) -> wkv7_time_mix_output
 * in one workgroup, with the same arithmetic and the same bf16 roundings in
 * the same order (the results are bit-identical to those three calls), but
 * without the intermediate w, k, v, a, b and y rows in memory and with one
 * launch instead of three.
 *
 * Replaces, for decode steps, the element-wise part of fla's RWKV7Attention
 * around the wkv call together with the call itself (external; reached
 * through the model forward, wkvm/runner/runner.py:80-88,
 * wkvm/models/rwkv7.py:108-113).
 *
 *   wkv_layer, num_rows, H, slot_ids, row_order, B, scale: as wkv7_decode_slots
 *   r, k, v, w_lora, a_lora, g        [B, H*64] bf16 projection / LoRA outputs
 *   v_lora, v_first                   [B, H*64] bf16, both NULL for the first layer
 *   k_k, k_a, r_k, ln_w, ln_b         [H*64] bf16 parameters; eps as wkv7_time_mix_output
 *   out                               [B, H*64] bf16: the output projection's input
 *   v_out                             [B, H*64] bf16 or NULL: the WKV op's v (the
 *                                     first layer's is v_first for the others)
 * Pointers must be 8-byte aligned (else WKV7_ERR_SHAPE).
 */
int wkv7_decode_block(float *wkv_layer, int64_t num_rows, int32_t H, const int32_t *slot_ids,
                      const int32_t *row_order, int32_t B, const uint16_t *r, const uint16_t *k,
                      const uint16_t *v, const uint16_t *w_lora, const uint16_t *a_lora,
                      const uint16_t *v_lora, const uint16_t *v_first, const uint16_t *g,
                      const uint16_t *k_k, const uint16_t *k_a, const uint16_t *r_k,
                      const uint16_t *ln_w, const uint16_t *ln_b, float eps, float scale,
                      uint16_t *out, uint16_t *v_out, void *stream);

/*
 * Grouped projection GEMMs of the RWKV-7 time-mix block, for few rows (decode
 * batches): up to WKV7_PROJ_MAX_GROUPS independent products in one launch,
 *     y_g[m][c] = act_g( sum_j x_g[m][j] w_g[c][j] + bias_g[c] ),
 * bf16 operands on the matrix cores, fp32 accumulation, bias and activation
 * on the fp32 sum, one bf16 rounding per output. All groups share the row
 * count m; each has its own k, n, pointers and strides.
 *
 * Replaces the nn.Linear calls of fla's RWKV7Attention (external; reached
 * through the model forward, wkvm/runner/runner.py:80-88): the r, k, v and o
 * projections (weights [out, in] as nn.Linear holds them) and both stages of
 * the w, a, v and g LoRAs, with the LoRAs' inner tanh and sigmoid fused into
 * the first stage's epilogue.
 *
 *   x     [m, k] bf16, row stride ldx elements (ldx >= k, ldx % 8 == 0)
 *   w     [n, k] bf16, row stride ldw elements (ldw >= k, ldw % 8 == 0)
 *   bias  [n] bf16, or NULL
 *   y     [m, n] bf16, row stride ldy elements (ldy >= n)
 * k must be a positive multiple of 32; x and w 16-byte aligned (else
 * WKV7_ERR_SHAPE). y must not overlap any group's x, w or bias.
 */
#define WKV7_PROJ_MAX_GROUPS 8
#define WKV7_ACT_NONE 0
#define WKV7_ACT_TANH 1
#define WKV7_ACT_SIGMOID 2

typedef struct wkv7_proj_group {
  const uint16_t *x;
  const uint16_t *w;
  const uint16_t *bias;
  uint16_t *y;
  int64_t ldx;
  int64_t ldw;
  int64_t ldy;
  int32_t n;
  int32_t k;
  int32_t act;
  int32_t reserved; /* set to 0 */
} wkv7_proj_group;

int wkv7_proj_grouped(int64_t m, const wkv7_proj_group *groups, int32_t ngroups,
                      void *workspace, size_t workspace_bytes, void *stream);

/* Workspace wkv7_proj_grouped can use for these products on the current
 * device (0: none). With at least this many bytes (16-byte aligned) it may
 * split long k over several workgroups, whose fp32 partials a second kernel
 * sums in a fixed order; with less it runs unsplit. Both give results within
 * one bf16 ulp of the exact product; each is deterministic. */
size_t wkv7_proj_workspace_bytes(int64_t m, const wkv7_proj_group *groups, int32_t ngroups);

/*
 * wkv7_proj_grouped with no workspace argument and no allocation of any kind:
 * when the launch splits k, the fp32 partials go to a library-owned static
 * device array of WKV7_PROJ_STATIC_SCRATCH_BYTES on each GPU (held until the
 * process ends; its address is looked up once per device, on the first call
 * made with that device current). Same products, same split decision and
 * bit-identical results as wkv7_proj_grouped given the workspace
 * wkv7_proj_workspace_bytes asks for.
 *
 * No counterpart in the reference. It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops and
 * harnesses that forbid hipMalloc.
 *
 * Limits: a split needing more than WKV7_PROJ_STATIC_SCRATCH_BYTES of
 * partials returns WKV7_ERR_WORKSPACE (nothing is enqueued); on a 256-unit
 * MI355X the split plan needs at most 4 MiB. Every call on one GPU shares
 * that GPU's array and leaves its partials there: calls that overlap on one
 * GPU (on different streams, or from several host threads) race. Each split
 * launch writes every partial it later sums, so nothing needs clearing.
 */
#define WKV7_PROJ_STATIC_SCRATCH_BYTES (8u * 1024u * 1024u)

int wkv7_proj_grouped_noalloc(int64_t m, const wkv7_proj_group *groups, int32_t ngroups,
                              void *stream);

#ifdef __cplusplus
}
#endif

#endif /* WKV7_H */
