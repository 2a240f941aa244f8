/*
 * koemi_hip.h — C ABI of the MI355X (gfx950) HERM hot-path kernels.
 *
 * Every entry point takes plain device pointers, element counts and an opaque
 * HIP stream (a hipStream_t passed as void*; NULL is the null stream). Inputs
 * are borrowed, outputs and workspaces are caller-allocated device memory. The
 * library never allocates device memory itself: operations that need scratch
 * space export a *_workspace_bytes() query and take a workspace pointer.
 *
 * All tensors are dense row-major and contiguous. Booleans are one byte
 * (0 or 1, the torch.bool layout). Every entry point returns KOEMI_OK (0) or a
 * KOEMI_ERR_* status; koemi_last_error() then returns a message for the
 * calling host thread. Work is enqueued asynchronously on `stream`.
 *
 * Reference interfaces (Koemi-5HOM, src/koemi/cuda_kernels/...) that each
 * group of entry points replaces are cited next to the declarations.
 */
#ifndef KOEMI_HIP_H
#define KOEMI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (the torch dtype each one mirrors in parentheses). */
enum koemi_dtype {
    KOEMI_F32 = 0,  /* torch.float32  */
    KOEMI_F16 = 1,  /* torch.float16  */
    KOEMI_BF16 = 2, /* torch.bfloat16 */
    KOEMI_F64 = 3,  /* torch.float64  */
    KOEMI_I32 = 4,  /* torch.int32    */
    KOEMI_I64 = 5,  /* torch.int64    */
    KOEMI_BOOL = 6  /* torch.bool     */
};

enum koemi_status {
    KOEMI_OK = 0,
    KOEMI_ERR_INVALID = 1,     /* argument violates the operator contract          */
    KOEMI_ERR_UNSUPPORTED = 2, /* dtype / size outside what this build implements  */
    KOEMI_ERR_LAUNCH = 3       /* the HIP runtime rejected a kernel launch          */
};

typedef void* koemi_stream_t;

/* ABI version, mirrors KOEMI_CUDA_ABI_VERSION = 1
 * (cuda_kernels/loader.py:32; core/rmsnorm_silu.cpp:74; moe/moe_kernels.cpp:257). */
int koemi_abi_version(void);

/* Message describing the last failure on the calling host thread ("" if none). */
const char* koemi_last_error(void);

/* ---------------------------------------------------------------- dense --- */
/* Replaces the pybind `forward(a, b, h0) -> h` of dense/affine_scan.cu:119-167
 * (front dense/affine_scan.py:51-98). h_t = a_t * h_{t-1} + b_t over t in
 * [0, sequence), h_{-1} = initial. increment/states are [batch, sequence,
 * features]; retention is the same shape, or [batch, sequence] when
 * broadcast_retention != 0; initial is [batch, features]. dtype is one of
 * F32/F16/BF16/F64; accumulation is fp32 (fp64 for F64). */
int koemi_affine_scan_forward(const void* retention, const void* increment, const void* initial,
                              void* states, int64_t batch, int64_t sequence, int64_t features,
                              int broadcast_retention, int dtype, koemi_stream_t stream);

/* Replaces the pybind `backward(a, h0, h, dh) -> (da, db, dh0)` of
 * dense/affine_scan.cu:169-226. grad_retention is always full shape
 * [batch, sequence, features]; the caller reduces it for broadcast retention
 * (dense/affine_scan.py:233-255). */
int koemi_affine_scan_backward(const void* retention, const void* initial, const void* states,
                               const void* grad_states, void* grad_retention, void* grad_increment,
                               void* grad_initial, int64_t batch, int64_t sequence,
                               int64_t features, int broadcast_retention, int dtype,
                               koemi_stream_t stream);

/* ----------------------------------------------------------------- core --- */
/* Replaces `rmsnorm_silu_forward(x, w, eps) -> [y, inverse_rms]` of
 * core/rmsnorm_silu.cpp:56-59 / rmsnorm_silu.cu:203-217.
 * inv = rsqrt(mean(x^2) + eps) per row (fp32), y = silu(x * inv * w).
 * x, y: [rows, hidden]; weight: [hidden]; dtype F32/F16/BF16. */
int koemi_rmsnorm_silu_forward(const void* input, const void* weight, void* output,
                               float* inverse_rms, int64_t rows, int64_t hidden, double eps,
                               int dtype, koemi_stream_t stream);

/* Replaces `rmsnorm_silu_backward(g, x, w, inv, eps) -> [dx, dw]` of
 * core/rmsnorm_silu.cpp:61-69 / rmsnorm_silu.cu:219-245. The weight gradient is
 * reduced deterministically in two stages (no atomics) through the workspace. */
size_t koemi_rmsnorm_silu_backward_workspace_bytes(int64_t rows, int64_t hidden);
int koemi_rmsnorm_silu_backward(const void* grad_output, const void* input, const void* weight,
                                const float* inverse_rms, void* grad_input, void* grad_weight,
                                int64_t rows, int64_t hidden, int dtype, void* workspace,
                                size_t workspace_bytes, koemi_stream_t stream);

/* ---------------------------------------------------------------- think --- */
/* Row kernel of think/surprise_kernel.cu:84-134 (`causal_surprise` forward
 * after its logits GEMM). For each row r with valid[r]:
 *   z_j = logits[r, j] (+ bias[j]),  nll = log(sum_j exp(z_j - max)) + max - z_t,
 *   surprise[r] = 1 - exp(-nll / log_vocab);   invalid rows -> 0.
 * logits fp32 [rows, vocab]; bias [vocab] of `dtype` or NULL; targets int64;
 * surprise [rows] of `dtype` (F32/F16/BF16). The summation order and the
 * exp/log routines are fixed (see surprise.hip), so results are reproducible
 * bit for bit. log_vocab is float(log(vocab)) as the reference computes it. */
int koemi_surprise_rows_forward(const float* logits, const void* bias, const int64_t* target_ids,
                                const uint8_t* valid_mask, void* surprise, int64_t rows,
                                int64_t vocab, float log_vocab, int dtype, koemi_stream_t stream);

/* Row kernel of think/surprise_kernel.cu:136-192: d logits for an upstream
 * gradient on surprise. grad_logits fp32 [rows, vocab]; invalid rows -> 0. */
int koemi_surprise_rows_backward(const float* logits, const void* bias, const int64_t* target_ids,
                                 const uint8_t* valid_mask, const void* grad_surprise,
                                 float* grad_logits, int64_t rows, int64_t vocab, float log_vocab,
                                 int dtype, koemi_stream_t stream);

/* Salience admission with a fixed threshold (model/network.py:349):
 * admission[i] = valid[i] && surprise[i] > threshold. surprise of `dtype`. */
int koemi_admission_threshold(const void* surprise, const uint8_t* valid_mask, uint8_t* admission,
                              int64_t count, float threshold, int dtype, koemi_stream_t stream);

/* Admission at a quantile of the scores: tau = torch.quantile(surprise, q)
 * with linear interpolation (rank = float(q) * (count - 1) in fp32), then
 * admission[i] = valid[i] && surprise[i] > tau. tau is written to
 * *threshold_out (device memory). Exact order-statistic selection on device,
 * no host round trip. surprise fp32, count >= 1. */
size_t koemi_admission_quantile_workspace_bytes(int64_t count);
int koemi_admission_quantile(const float* surprise, const uint8_t* valid_mask, uint8_t* admission,
                             float* threshold_out, int64_t count, float quantile, void* workspace,
                             size_t workspace_bytes, koemi_stream_t stream);

/* koemi_admission_quantile without a caller workspace and without any
 * allocation: no counterpart in the reference. It is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The partitioned select's records and
 * candidate slots live in a static device array of 263,424 bytes per GPU
 * (held until the process ends), enough for every count; counts needing more
 * are rejected (KOEMI_ERR_UNSUPPORTED). The array's device address is resolved
 * once per device on the first call there (hipGetSymbolAddress, with that
 * device current). Every call on one GPU shares its array, and nothing in it
 * needs to start at zero: calls on one GPU that overlap in time (different
 * streams without ordering) race and must not be issued. Same inputs, outputs
 * and results as koemi_admission_quantile. */
int koemi_admission_quantile_noalloc(const float* surprise, const uint8_t* valid_mask, uint8_t* admission,
                                     float* threshold_out, int64_t count, float quantile,
                                     koemi_stream_t stream);

/* ------------------------------------------------------------------ moe --- */
/* Replaces `route_topk(tok, prev, valid, E, k)` of moe/moe_kernels.cpp:193-201
 * with the int64 semantics of the PyTorch oracle (model/experts.py:283-289):
 * h = mix32(tok * 1000003 + prev * 97409); a[t, s] = (h + s * 0x9E3779B9) mod E
 * for valid tokens, -1 otherwise. ids are I32 or I64 (`id_dtype`).
 * *duplicate_flag (device int32, caller-zeroed) is set to 1 when a valid token
 * received the same expert in two slots (moe/__init__.py:113-125, 171-175);
 * NULL skips the check. */
int koemi_moe_route_hash(const void* token_ids, const void* previous_token_ids,
                         const uint8_t* valid_mask, int id_dtype, int64_t* assignments,
                         int32_t* duplicate_flag, int64_t tokens, int64_t expert_count,
                         int64_t top_k, koemi_stream_t stream);

/* The synthetic "token id mod E" route of the benchmark's C4 hash variant
 * (BASELINE configs[3]); no counterpart in the reference, whose hash route is
 * koemi_moe_route_hash above. a[t, s] = (tok[t] + s) mod E (torch.remainder
 * sign: in [0, E) for negative ids) for valid tokens, -1 otherwise; ids are
 * I32 or I64. Slots never repeat an expert (s < E). */
int koemi_moe_route_modulo(const void* token_ids, const uint8_t* valid_mask, int id_dtype,
                           int64_t* assignments, int64_t tokens, int64_t expert_count, int64_t top_k,
                           koemi_stream_t stream);

/* Learned top-k gate of model/router.py:46-49: p = softmax(logits) in fp32,
 * (weights, assignments) = topk(p, k) in descending order, ties to the lower
 * expert index; invalid tokens get assignment -1 and weight 0.
 * router_logits fp32 [tokens, expert_count], expert_count <= 1024. */
int koemi_moe_route_learned(const float* router_logits, const uint8_t* valid_mask,
                            int64_t* assignments, float* weights, int64_t tokens,
                            int64_t expert_count, int64_t top_k, koemi_stream_t stream);

/* LearnedExpertMixture.forward's route with its RouterStatistics
 * (model/router.py:11-22, 43-59): assignments and weights as
 * koemi_moe_route_learned (the same bits), and, as device fp32 values,
 * probability_mass [expert_count] = the sum of the valid tokens' softmax
 * probabilities, assignment_counts [expert_count] = the valid assignments per
 * expert (exact integers), valid_count [1] = the number of valid tokens, and
 * (balance_loss != NULL) balance_loss [1] = RouterStatistics.balance_loss,
 * E * sum_e (mass_e / max(valid, 1)) * (counts_e / max(sum counts, 1)).
 * Sums run in a fixed order (tokens in workgroups of 256, then workgroups in
 * order), so the results do not depend on timing. Workspace:
 * koemi_moe_route_learned_stats_workspace_bytes(tokens, expert_count) bytes;
 * no zeroing needed. tokens == 0 gives zero statistics. */
size_t koemi_moe_route_learned_stats_workspace_bytes(int64_t tokens, int64_t expert_count);
int koemi_moe_route_learned_stats(const float* router_logits, const uint8_t* valid_mask, int64_t* assignments,
                                  float* weights, float* probability_mass, float* assignment_counts,
                                  float* valid_count, float* balance_loss, int64_t tokens, int64_t expert_count,
                                  int64_t top_k, void* workspace, size_t workspace_bytes, koemi_stream_t stream);

/* RouterStatistics.balance_loss (model/router.py:17-22) of given statistics
 * (e.g. merged over windows by merge_router_statistics, router.py:25-32), in
 * fp32 and expert order, as koemi_moe_route_learned_stats computes it. */
int koemi_moe_router_balance_loss(const float* probability_mass, const float* assignment_counts,
                                  const float* valid_count, int64_t expert_count, float* balance_loss,
                                  koemi_stream_t stream);

/* Contract checks of moe/__init__.py:113-125, 213-220 on device:
 * flags[0] |= 1 if a valid assignment is outside [0, expert_count),
 * flags[1] |= 1 if a valid token repeats an expert. flags: caller-zeroed int32[2]. */
int koemi_moe_check_assignments(const void* assignments, int assignment_dtype,
                                const uint8_t* valid_mask, int32_t* flags, int64_t tokens,
                                int64_t top_k, int64_t expert_count, koemi_stream_t stream);

/* Per-expert activation counts (model/network.py:48-70):
 * counts[e] = #{(t, s): valid[t] && assignments[t, s] == e}. counts int64 [E]
 * (overwritten; no zeroing needed). */
int koemi_moe_expert_counts(const void* assignments, int assignment_dtype,
                            const uint8_t* valid_mask, int64_t* counts, int64_t tokens,
                            int64_t top_k, int64_t expert_count, koemi_stream_t stream);

/* Replaces `permute_topk(ctx, assignments, valid, E)` of
 * moe/moe_kernels.cu:390-499: pair key = expert (E for an invalid token, an
 * out-of-range expert or a repeated slot); pairs are stably sorted by key;
 * segment_offsets[E + 1] is the exclusive prefix of the per-expert counts
 * (segment_offsets[E] = valid pairs); sorted_rows = pair / top_k;
 * sorted_experts = key; sorted_context[i] = context[sorted_rows[i]] for
 * i < segment_offsets[E], zero afterwards. pair_weights [tokens, top_k] fp32
 * (or NULL) is permuted the same way into sorted_weights (0 past the valid
 * pairs). Context dtype F32/F16/BF16; assignments I32/I64. expert_count <= 4095.
 * sorted_context may be NULL: only the indices are formed (for
 * koemi_moe_grouped_mlp_indexed, which reads the context rows by sorted_rows). */
/* The index phase of koemi_moe_permute alone (no context; a build-side entry
 * for the HERM block), which also hands over its pair -> position map:
 * pair_positions[t * top_k + s] = the sorted position of pair (t, s) (valid
 * pairs below segment_offsets[E]). Same workspace as koemi_moe_permute. */
/* koemi_moe_route_hash followed by koemi_moe_permute_indices in the same
 * launches, the assignments never stored (a build-side entry for the HERM
 * block's hash-routed experts): each pair's expert is hashed from its token
 * and previous token inside the permutation. The same outputs as those two
 * calls. ids I32 or I64 (id_dtype); the workspace of
 * koemi_moe_permute_workspace_bytes. */
int koemi_moe_permute_hash_indices(const void* token_ids, const void* previous_token_ids, int id_dtype,
                                   const uint8_t* valid_mask, int64_t* sorted_rows, int64_t* sorted_experts,
                                   int64_t* segment_offsets, int64_t* pair_positions, int64_t tokens, int64_t top_k,
                                   int64_t expert_count, void* workspace, size_t workspace_bytes,
                                   koemi_stream_t stream);
int koemi_moe_permute_indices(const void* assignments, int assignment_dtype, const uint8_t* valid_mask,
                              const float* pair_weights, int64_t* sorted_rows, int64_t* sorted_experts,
                              int64_t* segment_offsets, float* sorted_weights, int64_t* pair_positions,
                              int64_t tokens, int64_t top_k, int64_t expert_count, void* workspace,
                              size_t workspace_bytes, koemi_stream_t stream);
size_t koemi_moe_permute_workspace_bytes(int64_t tokens, int64_t top_k, int64_t expert_count);
int koemi_moe_permute(const void* context, int context_dtype, const void* assignments,
                      int assignment_dtype, const uint8_t* valid_mask, const float* pair_weights,
                      void* sorted_context, int64_t* sorted_rows, int64_t* sorted_experts,
                      int64_t* segment_offsets, float* sorted_weights, int64_t tokens,
                      int64_t width, int64_t top_k, int64_t expert_count, void* workspace,
                      size_t workspace_bytes, koemi_stream_t stream);

/* Replaces `grouped_expert_mlp(...)` of moe/moe_kernels.cu:501-558: for each
 * sorted pair i < segment_offsets[E] with expert e = sorted_experts[i]:
 *   y_i = W_o[e] (silu(W_g[e] x_i + b_g[e]) * (W_v[e] x_i + b_v[e])) + b_o[e];
 * rows past the valid pairs are zero. Weights: gate/value [E, hidden, width],
 * their biases [E, hidden], output [E, width, hidden], its bias [E, width].
 * BF16 runs on bf16 MFMA (fp32 accumulation, the GLU product rounded to bf16
 * between the two GEMMs); F32/F16 run a fp32-accumulating scalar path.
 * The tile scheduler reads segment_offsets on device (no host sync). */
size_t koemi_moe_grouped_mlp_workspace_bytes(int64_t pairs, int64_t width, int64_t hidden,
                                             int64_t expert_count, int dtype);
int koemi_moe_grouped_mlp(const void* sorted_context, const int64_t* sorted_experts,
                          const int64_t* segment_offsets, const void* gate_weights,
                          const void* gate_biases, const void* value_weights,
                          const void* value_biases, const void* output_weights,
                          const void* output_biases, void* output, int64_t pairs, int64_t width,
                          int64_t hidden, int64_t expert_count, int dtype, void* workspace,
                          size_t workspace_bytes, koemi_stream_t stream);

/* koemi_moe_grouped_mlp without the sorted copy of the context (no
 * counterpart in the reference, whose permute_topk always gathers it): pair i
 * reads row sorted_rows[i] (clamped to [0, tokens)) of context [tokens,
 * width], as koemi_moe_permute's sorted_rows gives it, straight into the first
 * GEMM's operand tiles. bf16 only, width and hidden multiples of 64, 16-byte
 * aligned operands, tokens * width < 2^31; the workspace of
 * koemi_moe_grouped_mlp_workspace_bytes(pairs, width, hidden, expert_count,
 * KOEMI_BF16). The rows of the valid pairs equal koemi_moe_grouped_mlp's
 * on the gathered context bit for bit; the rows past them (pairs >=
 * segment_offsets[E]) are not written. */
int koemi_moe_grouped_mlp_indexed(const void* context, int64_t tokens, const int64_t* sorted_rows,
                                  const int64_t* segment_offsets, const void* gate_weights, const void* gate_biases,
                                  const void* value_weights, const void* value_biases, const void* output_weights,
                                  const void* output_biases, void* output, int64_t pairs, int64_t width,
                                  int64_t hidden, int64_t expert_count, void* workspace, size_t workspace_bytes,
                                  koemi_stream_t stream);

/* Expert weights in fragment order, for koemi_moe_grouped_mlp_fragments (no
 * counterpart in the reference, whose grouped_expert_mlp of
 * moe/moe_kernels.cu:501-558 reads row-major weights): weights [matrices,
 * rows, cols] bf16 (rows a multiple of 32, cols of 64; e.g. the gate weights
 * [E, hidden, width] as E x hidden rows) into fragments of the same size,
 * each 32-row block stored as [cols / 64][4][64][8]: element (32 b + r, c)
 * goes to block b at ((c / 64) * 4 + (c % 32) / 8) * 512 + (32 * ((c % 64) /
 * 32) + r) * 8 + c % 8. Not in place; 16-byte aligned. */
int koemi_moe_weights_to_fragments(const void* weights, void* fragments, int64_t matrices, int64_t rows,
                                   int64_t cols, koemi_stream_t stream);

/* koemi_moe_grouped_mlp_indexed for a few rows per expert (a decode step:
 * pairs <= 64 * expert_count, KOEMI_ERR_UNSUPPORTED otherwise) with the
 * three weight tensors in fragment order (koemi_moe_weights_to_fragments of
 * gate and value [E, hidden, width] and output [E, width, hidden]; biases as
 * they are): every weight load of the kernels reads contiguous memory. Same
 * arguments, workspace and results as koemi_moe_grouped_mlp_indexed, bit for
 * bit (the same products in the same order). */
int koemi_moe_grouped_mlp_fragments(const void* context, int64_t tokens, const int64_t* sorted_rows,
                                    const int64_t* segment_offsets, const void* gate_fragments,
                                    const void* gate_biases, const void* value_fragments, const void* value_biases,
                                    const void* output_fragments, const void* output_biases, void* output,
                                    int64_t pairs, int64_t width, int64_t hidden, int64_t expert_count,
                                    void* workspace, size_t workspace_bytes, koemi_stream_t stream);

/* Salient-memory ring update, LocalKeyValueMemory.salient_tail of
 * model/memory.py:431-455. Per batch row, the carried entries [S] followed by
 * the window's entries [L] (keys/values [*, D] of `dtype`, validity = carried
 * valid flags then the admission mask). When S + L <= capacity the outputs are
 * the concatenation ([B, S + L, D], flags unchanged). Otherwise the outputs
 * are [B, capacity, D]: the latest min(#valid, capacity) valid entries in time
 * order, and — when fewer than capacity are valid — the latest invalid entries
 * as filler, all in ascending time order, with the keys and values of invalid
 * slots zeroed. (The reference takes torch.topk over ranks valid ? t : -1;
 * which tied invalid filler it picks is unspecified, so this rule fixes it.)
 * capacity <= 4096. */
int koemi_salient_tail(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                       const void* keys, const void* values, const uint8_t* admission, void* out_keys,
                       void* out_values, uint8_t* out_valid, int64_t batch, int64_t carried, int64_t length,
                       int64_t width, int64_t capacity, int dtype, koemi_stream_t stream);

/* The rings a sequence-parallel prefill needs (no single reference op: the
 * state that forward_parallel carries from window to window, network.py:
 * 176-197, through LocalKeyValueMemory.tail and salient_tail, memory.py:
 * 385-403, 431-455). For each batch row and r = 0 .. length / window, the ring
 * as it stands before position r * window of the sequence: entries = the
 * carried ring [carried] followed by positions 0 .. r * window - 1, each with
 * its flag. tail != 0: the last `capacity` entries with their flags, rows as
 * stored (the local ring; flags = valid). tail == 0: the salient_tail rule
 * above (flags = admission; invalid slots zeroed). The rings carried into the
 * windows r < length / window go to out_* ([batch * length / window,
 * capacity, width] keys and values, [batch * length / window, capacity]
 * flags; row b * (length / window) + r), the ring after the whole sequence
 * to final_* ([batch, capacity, ...]). Requires carried >= capacity (a static
 * ring, state.py:43-76) and length % window == 0.
 * The sequence's keys and values are rows key_row_stride elements apart
 * (0: width) of key_dtype: dtype itself, or KOEMI_BF16 into fp32 rings (the
 * bf16 columns of the block's key/value projection read in place, widened
 * exactly). key_valid (optional, [batch, length]): a position whose byte is
 * 0 enters the ring with zero key and value, which is the reference's masking
 * of the projected keys and values by the validity mask (network.py:337-340)
 * done on the way (reads need no such masking: only valid entries are ever
 * eligible). out_keys, out_values and out_valid all NULL: only the final
 * ring is built (LocalKeyValueMemory.tail or salient_tail of one window), of
 * min(carried + length, capacity) slots, any carried >= 0. Entries of
 * another dtype, stride or with key_valid require fp32 rings. */
int koemi_window_rings(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                       const void* keys, const void* values, int key_dtype, int64_t key_row_stride,
                       const uint8_t* key_valid, const uint8_t* flags, void* out_keys, void* out_values,
                       uint8_t* out_valid, void* final_keys, void* final_values, uint8_t* final_valid, int64_t batch,
                       int64_t carried, int64_t length, int64_t window, int64_t width, int64_t capacity, int tail,
                       int dtype, koemi_stream_t stream);

/* The local and the salient read of a one-position window (a decode step,
 * network.py:337-358: LocalKeyValueMemory.read_window and
 * read_salient_window with one query) in one launch: each query [batch, width]
 * attends, with scores key . query / sqrt(width), to the valid carried slots
 * of each ring (for the local ring only the newest `window` slots), zero
 * output when none is eligible. fp32, width % 4 == 0, at most 256 slots per
 * ring, 16-byte aligned rows. Results equal koemi_local_read and
 * koemi_salient_read with length 1. */
int koemi_read_step_pair(const float* local_keys, const float* local_values, const uint8_t* local_valid,
                         int64_t local_slots, int64_t window, const float* salient_keys, const float* salient_values,
                         const uint8_t* salient_valid, int64_t salient_slots, const float* queries, float* local_out,
                         float* salient_out, int64_t batch, int64_t width, koemi_stream_t stream);

/* koemi_read_step_pair and the two rings after the position in the same
 * launch (a decode step's memory: network.py:337-358, 410-414 with
 * LocalKeyValueMemory.tail and salient_tail, memory.py:385-403, 431-455):
 * next_local_* = the last local_slots entries of [local ring ; entry] with
 * their valid bytes, rows as stored; next_salient_* = the salient_tail rule
 * of koemi_salient_tail over [salient ring ; entry] with capacity
 * salient_slots and the admission byte as the entry's flag (invalid slots
 * zeroed). The entry of batch row b is row b of keys / values (key_dtype
 * KOEMI_F32 or KOEMI_BF16, rows key_row_stride elements apart, 0: width;
 * the block's projection read in place), zeroed where valid[b] == 0
 * (network.py:337-340). Static rings (both slot counts >= 1); the next
 * rings must not overlap the carried ones. */
int koemi_read_step_pair_rings(const float* local_keys, const float* local_values, const uint8_t* local_valid,
                               int64_t local_slots, int64_t window, const float* salient_keys,
                               const float* salient_values, const uint8_t* salient_valid, int64_t salient_slots,
                               const float* queries, float* local_out, float* salient_out, const void* keys,
                               const void* values, int key_dtype, int64_t key_row_stride, const uint8_t* valid,
                               const uint8_t* admission, float* next_local_keys, float* next_local_values,
                               uint8_t* next_local_valid, float* next_salient_keys, float* next_salient_values,
                               uint8_t* next_salient_valid, int64_t batch, int64_t width, koemi_stream_t stream);

/* A decode step's whole memory in one launch: koemi_read_step_pair_rings
 * with the entries read from `projections` (rows row_stride elements apart
 * of projection_dtype, KOEMI_F32 or KOEMI_BF16: local keys at column
 * key_offset, local values at value_offset), and the one-position
 * associative read and update of koemi_assoc_scan_read (memory.py:82-144,
 * 244-255; network.py:734-740) on the same rows: value pre-activations at
 * assoc_value_offset, the key's and the query's feature logits at
 * feature_offset and query_feature_offset (`features` <= 32 columns each),
 * the decay and write logits at decay_offset and write_offset; surprise
 * [batch], the carried basis [batch, width, features] and normalizer
 * [batch, features] in, the read [batch, width] and the next basis and
 * normalizer out. The results equal the two separate entries'. */
int koemi_decode_memory_step(const float* local_keys, const float* local_values, const uint8_t* local_valid,
                             int64_t local_slots, int64_t window, const float* salient_keys,
                             const float* salient_values, const uint8_t* salient_valid, int64_t salient_slots,
                             const float* queries, float* local_out, float* salient_out, const void* projections,
                             int projection_dtype, int64_t row_stride, int64_t key_offset, int64_t value_offset,
                             const uint8_t* valid, const uint8_t* admission, float* next_local_keys,
                             float* next_local_values, uint8_t* next_local_valid, float* next_salient_keys,
                             float* next_salient_values, uint8_t* next_salient_valid, int64_t assoc_value_offset,
                             int64_t feature_offset, int64_t query_feature_offset, int64_t decay_offset,
                             int64_t write_offset, const float* surprise, const float* basis, const float* normalizer,
                             float* assoc_read, float* next_basis, float* next_normalizer, int64_t features,
                             int64_t batch, int64_t width, koemi_stream_t stream);

/* Bounded recurrent gates, BoundedRecurrentState.gates of model/memory.py:14-30
 * with the masking of network.py:306-309 (a torch composite in the
 * reference): for input rows u (rows x width, `dtype`),
 *   retention = sigmoid(u W_r^T + b_r), a = 2^-8 + (1 - 2^-7) retention,
 *   b = (1 - a) tanh(u W_c^T + b_c),
 * and where `valid` (one byte per row, may be NULL) is 0: a = 1, b = 0.
 * W_r, W_c are width x width (out x in), biases width; a and b are rows x width
 * in `dtype`. Products accumulate in fp32. width % 4 == 0. */
size_t koemi_recurrent_gates_workspace_bytes(int64_t rows, int64_t width);
int koemi_recurrent_gates(const void* input, const void* retention_weight, const void* retention_bias,
                          const void* candidate_weight, const void* candidate_bias, const uint8_t* valid,
                          void* retention_out, void* increment_out, int64_t rows, int64_t width, int dtype,
                          void* workspace, size_t workspace_bytes, koemi_stream_t stream);

/* The bounded recurrent state over a window in one call, fp32: the gates of
 * model/memory.py:14-30 with the masking of network.py:306-309 followed by the
 * affine scan of network.py:310 (h_t = a_t h_{t-1} + b_t from `initial`),
 * the gates formed in registers inside the scan rather than written to memory.
 * input [batch, length, width], weights width x width (out x in), biases
 * width, valid [batch, length] bytes or NULL, initial [batch, width], states
 * [batch, length, width]. The workspace is
 * koemi_recurrent_gates_workspace_bytes(batch * length, width). Results equal
 * koemi_recurrent_gates followed by koemi_affine_scan_forward. width % 4 == 0. */
int koemi_recurrent_scan(const float* input, const float* retention_weight, const float* retention_bias,
                         const float* candidate_weight, const float* candidate_bias, const uint8_t* valid,
                         const float* initial, float* states, int64_t batch, int64_t length, int64_t width,
                         void* workspace, size_t workspace_bytes, koemi_stream_t stream);

/* The same gates and scan from precomputed pre-activations (fp32, or bf16: a
 * GEMM's own output dtype, as nn.Linear under bf16 autocast), for callers
 * that form u W_r^T and u W_c^T themselves (one stacked GEMM): row r of the
 * batch x length rows holds the retention pre-activations at
 * preactivations[r * row_stride + retention_offset + f] and the candidate ones
 * at [... + candidate_offset + f], f < width. The biases (width each) are
 * added first; NULL means none (already inside the pre-activations). Then
 * a = 2^-8 + (1 - 2^-7) sigmoid, b = (1 - a) tanh, the valid mask (NULL: all
 * valid) and h_t = a_t h_{t-1} + b_t from `initial` [batch, width] into
 * `states` [batch, length, width], as in network.py:306-310; with
 * `states_bf16` (NULL: none) also a bf16 copy of the states for the next
 * projection's GEMM, rows bf16_row_stride elements apart (0: width).
 * `workspace` (NULL: none, else at least
 * koemi_gated_scan_workspace_bytes) lets a batch of a few long rows run as a
 * two-phase scan: the transfers of every 8-step segment first, then chunks of
 * the sequence in parallel, each from its carry composed through the segments
 * before it in order, which gives the same bits as the one-pass scan. */
size_t koemi_gated_scan_workspace_bytes(int64_t batch, int64_t length, int64_t width);
int koemi_gated_scan(const void* preactivations, int preactivation_dtype, int64_t row_stride,
                     int64_t retention_offset, int64_t candidate_offset, const float* retention_bias, const float* candidate_bias,
                     const uint8_t* valid, const float* initial, float* states, void* states_bf16,
                     int64_t bf16_row_stride, int64_t batch, int64_t length, int64_t width, void* workspace,
                     size_t workspace_bytes, koemi_stream_t stream);

/* BoundedRecurrentState.gates (model/memory.py:14-30: the projections
 * W_r u + b_r and W_c u + b_c, sigmoid retention and tanh candidate), the
 * masking of network.py:307-309 and the scan of network.py:310 in one kernel,
 * for bf16 inputs under autocast (the projection's results rounded to bf16
 * after the bias, as the reference's autocast GEMM writes them). inputs
 * [batch * length, input_width] bf16 (rows (b, t), contiguous); weights
 * [2 * width, input_width] bf16: the retention rows, then the candidate rows;
 * biases [2 * width] bf16 in the same order, or NULL. valid [batch, length]
 * (NULL: all valid), initial [batch, width] fp32; writes states [batch,
 * length, width] fp32, with states_bf16 (NULL: none) a bf16 copy whose rows
 * are bf16_row_stride elements apart (0: width), and with final_states (NULL:
 * none) the last position's states again as [batch, width] (the carried
 * state). The projection runs on
 * bf16 MFMA in tiles of 256 positions x 128 features, whose epilogue forms
 * the gates and scans them, so the pre-activations never reach memory; each
 * tile publishes its transfer (the affine map of its positions) and takes
 * its carry by applying the earlier tiles' transfers to the initial state in
 * order (bounded waits; the result does not depend on timing). Needs length % 256 == 0, width % 128 == 0,
 * input_width % 64 == 0 and 16-byte aligned inputs and weights
 * (KOEMI_ERR_UNSUPPORTED otherwise: take a GEMM and koemi_gated_scan), and a
 * workspace of koemi_gated_projection_scan_workspace_bytes(batch, length,
 * width) bytes (0 for unsupported shapes). Calls sharing one workspace must
 * not overlap in time.
 *
 * Every wait for an earlier tile's transfer is bounded by spin_limit polls
 * (0: the default, 2^22). A wait that runs out sets *status to 1 (a device
 * int32 the kernel never clears: the caller zeroes it and reads it after the
 * launch has completed; NULL: the workspace's word at byte offset 1024,
 * cleared by every launch) and makes that tile's carry NaN, so its states,
 * the final states and everything computed from them are NaN, never silently
 * wrong; the launch itself returns KOEMI_OK, as the failure is only known on
 * the device. spin_limit | KOEMI_GP_WITHHOLD_TRANSFERS makes no tile publish
 * its transfer, so every tile past the first of its sequence times out after
 * (spin_limit & ~KOEMI_GP_WITHHOLD_TRANSFERS) polls: the host's way to test
 * the timeout path with every wave still exiting normally. */
#define KOEMI_GP_WITHHOLD_TRANSFERS 0x80000000u
size_t koemi_gated_projection_scan_workspace_bytes(int64_t batch, int64_t length, int64_t width);
int koemi_gated_projection_scan(const void* inputs, const void* weights, const void* biases, const uint8_t* valid,
                                const float* initial, float* states, void* states_bf16, int64_t bf16_row_stride,
                                float* final_states, int64_t batch, int64_t length, int64_t width, int64_t input_width, void* workspace,
                                size_t workspace_bytes, int32_t* status, uint32_t spin_limit, koemi_stream_t stream);

/* nn.Linear over a few rows with bf16 weights (the HERM block's projections
 * in a decode step: the gate, working-state, fusion and head layers of
 * model/network.py:296-441 and model/memory.py, which the reference runs as
 * torch linear layers under bf16 autocast):
 *   output[r, n] = sum_k bf16(x[r, k]) * weight[n, k] + bias[n],
 * fp32 accumulation and results. x is `pieces` (1..4) row-major blocks
 * [rows, piece_width] of `input_dtype` (float32, rounded to bf16 on load, or
 * bfloat16) that together form K = pieces * piece_width, block i holding
 * columns [i * piece_width, (i + 1) * piece_width) (network.py:401-405
 * concatenates four such inputs); unused piece pointers may be NULL. weight
 * is [out_features, K] bf16, bias [out_features] fp32 or NULL, output
 * [rows, out_features] fp32. piece_width % 64 == 0, and % 1024 == 0 when
 * pieces > 1; any rows (each 64-row pass streams the weights once). */
int koemi_linear_rows(const void* input0, const void* input1, const void* input2, const void* input3, int pieces,
                      int64_t piece_width, int input_dtype, const void* weight, const float* bias, float* output,
                      int64_t rows, int64_t out_features, koemi_stream_t stream);

/* A decode step's gate projections with the gates and the one-position scan
 * in the epilogue (memory.py:14-30, network.py:306-310; nn.Linear then
 * BoundedRecurrentState.gates and one scan step in the reference):
 * weight [2 width, in_features] bf16 stacks the retention rows over the
 * candidate rows (no GEMM bias); with zr, zc the two products of row r's
 * input (rounded to bf16, as koemi_linear_rows), states[r, f] = a
 * initial[r, f] + b where (a, b) are the gates of zr + retention_bias[f] and
 * zc + candidate_bias[f] (biases fp32 or NULL), a = 1, b = 0 where
 * valid[r] == 0 (valid NULL: all valid); states_bf16 (NULL: none) receives
 * the bf16 copy, rows bf16_row_stride apart. Equal to koemi_linear_rows then
 * koemi_gated_scan at length 1. in_features % 64 == 0. */
int koemi_linear_rows_gated(const void* input, int input_dtype, const void* weight, const float* retention_bias,
                            const float* candidate_bias, const uint8_t* valid, const float* initial, float* states,
                            void* states_bf16, int64_t bf16_row_stride, int64_t rows, int64_t width,
                            int64_t in_features, koemi_stream_t stream);

/* koemi_linear_rows with K split over `splits` workgroup columns (a decode
 * step's 4096-wide fusion layer, network.py:401-405, spread over the chip):
 * block s of `partials` ([splits, rows, out_features] fp32) = the products
 * of K values [s K / splits, (s + 1) K / splits), the bias (fp32 or NULL)
 * added to block 0 only; the sum of the blocks in order is the projection
 * (koemi_herm_rmsnorm_parts adds them). piece_width % 1024 == 0 and
 * K / splits a multiple of 512 (fp32 inputs) or 1024 (bf16 inputs). */
int koemi_linear_rows_split(const void* input0, const void* input1, const void* input2, const void* input3,
                            int pieces, int64_t piece_width, int input_dtype, const void* weight, const float* bias,
                            float* partials, int64_t rows, int64_t out_features, int splits, koemi_stream_t stream);

/* `count` (1..32) independent koemi_linear_rows projections of one shape in
 * one launch (a decode step's content heads of every layer, network.py:
 * 318-325, 677-698, each on its own layer's carried working state):
 * output[e] ([rows, out_features] fp32 blocks, one after another) =
 * bf16(inputs[e]) weights[e]^T + biases[e]; inputs[e] [rows, in_features] of
 * input_dtype, weights[e] [out_features, in_features] bf16, `biases` NULL or
 * an array whose entries may be NULL. The pointer arrays are host arrays,
 * read during the call. in_features % 64 == 0. */
int koemi_linear_rows_batched(const void* const* inputs, int input_dtype, const void* const* weights,
                              const float* const* biases, float* output, int count, int64_t rows,
                              int64_t in_features, int64_t out_features, koemi_stream_t stream);

/* Salient-memory read, LocalKeyValueMemory.read_salient_window of
 * model/memory.py:405-429 (called at network.py:350-358; a torch composite in
 * the reference). For every batch row b and query t < length:
 *   slots = [carried entries (carried) ; window entries (length)],
 *   score_s = key_s . query_t / sqrt(width),
 *   eligible: carried slot s with carried_valid[b, s], window slot j with
 *   admission[b, j] and j < t,
 *   out[b, t] = softmax over the eligible slots applied to the values (zero
 *   when no slot is eligible).
 * Keys, values and queries are [batch, *, width] in `dtype`, the masks bytes
 * (0/1); out is [batch, length, width] in `dtype`. Products accumulate in fp32.
 * carried may be 0 (carried pointers may then be NULL). */
size_t koemi_salient_read_workspace_bytes(int64_t batch, int64_t carried, int64_t length, int64_t width,
                                          int dtype);
int koemi_salient_read(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                       const void* keys, const void* values, const uint8_t* admission, const void* queries,
                       void* out, int64_t batch, int64_t carried, int64_t length, int64_t width, int dtype,
                       void* workspace, size_t workspace_bytes, koemi_stream_t stream);

/* Associative memory of one HERM block window: HierarchicalAssociativeMemory.
 * project (the feature softmax, value tanh, bounded decay and write weight),
 * query_features, fast_write_terms and scan_and_read of model/memory.py:82-144,
 * 244-255, with the write masking of network.py:734-740 (torch composites in
 * the reference). `projections` is [batch * length, row_stride] in
 * projection_dtype (KOEMI_F32 or KOEMI_BF16: a bf16 GEMM's own output),
 * at the given column offsets, the value pre-activations (width columns), the
 * feature logits W_f key + b_f and W_f query + b_f (features columns each)
 * and the decay and write logits (one column each); surprise fp32 and valid
 * bytes [batch * length]; basis fp32 [batch, width, features], normalizer
 * [batch, features]. Writes the reads (read_dtype KOEMI_F32 or KOEMI_BF16,
 * rows read_row_stride elements apart, 0: width; a one-position window only
 * fp32 contiguous) and the window's
 * final basis and normalizer (fp32); next_basis and next_normalizer must not
 * alias basis and normalizer. features <= 32; the window length is bounded by
 * LDS (at most 480 positions with 16 features, 384 with 32). A window of one
 * position (a decode step) needs no workspace; longer ones take
 * koemi_assoc_scan_read_workspace_bytes(batch, length, width, features)
 * bytes for the per-position weights (features, cumulative log-decays, write
 * weights) that three launches share: prepare, state, reads. */
size_t koemi_assoc_scan_read_workspace_bytes(int64_t batch, int64_t length, int64_t width, int64_t features);
int koemi_assoc_scan_read(const void* projections, int projection_dtype, int64_t row_stride, int64_t value_offset,
                          int64_t feature_offset, int64_t query_feature_offset, int64_t decay_offset, int64_t write_offset,
                          const float* surprise, const uint8_t* valid, const float* basis, const float* normalizer,
                          void* read, int read_dtype, int64_t read_row_stride, float* next_basis,
                          float* next_normalizer, int64_t batch, int64_t length, int64_t width, int64_t features,
                          void* workspace, size_t workspace_bytes, koemi_stream_t stream);

/* koemi_assoc_scan_read over a whole sequence of `windows` windows of
 * `window` positions at once (forward_parallel, network.py:176-197, carrying
 * the memory state from window to window): the same layouts with length =
 * windows * window. Four launches: every window's per-position weights and
 * its own terms of the final state from a zero carried state, a scan over the
 * windows of state' = e^{c_{L-1}} state + terms (the one-window update, so
 * each window's carried state equals a window-by-window run's), and the reads
 * of every window from its carried state (the one-window read kernel, so the
 * reads equal a window-by-window run's bit for bit). Writes the reads [batch,
 * length, width] and the state after the last window. window >= 2; workspace
 * of koemi_assoc_scan_read_windows_workspace_bytes(batch, windows, window,
 * width, features) bytes. */
size_t koemi_assoc_scan_read_windows_workspace_bytes(int64_t batch, int64_t windows, int64_t window, int64_t width,
                                                     int64_t features);
int koemi_assoc_scan_read_windows(const void* projections, int projection_dtype, int64_t row_stride,
                                  int64_t value_offset,
                                  int64_t feature_offset, int64_t query_feature_offset, int64_t decay_offset,
                                  int64_t write_offset, const float* surprise, const uint8_t* valid,
                                  const float* basis, const float* normalizer, void* read, int read_dtype,
                                  int64_t read_row_stride, float* next_basis, float* next_normalizer, int64_t batch,
                                  int64_t windows, int64_t window, int64_t width, int64_t features, void* workspace,
                                  size_t workspace_bytes, koemi_stream_t stream);

/* The refine memory of the herm ablation (model/network.py:359-384; the write
 * terms of memory.py:257-268, masked as network.py:733-739; scan_and_read of
 * memory.py:97-144 over the refine basis and normalizer). The projections and
 * their column layout are those of koemi_assoc_scan_read (features, query
 * features, decay and write logits, value pre-activations); per position the
 * refine terms are decay' = min(1 - (1 - decay) refine_decay_rate, 1 - 2^-16),
 * weight' = sigmoid(w) clamp(surprise, 0, 1) clamp(novelty, 0, 1) (novelty
 * [batch, length] fp32, from koemi_local_novelty) and value' =
 * clamp(tanh(v) - fast_read, -2, 2), fast_read being the position's fast
 * associative read ([batch, length, width] of fast_dtype F32 or BF16, rows
 * fast_row_stride apart; 0: width); invalid positions decay 1, weight 0.
 * Reads go to `read` and the next refine state to next_basis /
 * next_normalizer as for koemi_assoc_scan_read (a one-position window takes
 * and writes contiguous fp32). Workspace:
 * koemi_assoc_refine_scan_read_workspace_bytes (the prepared weights and the
 * refine values). */
size_t koemi_assoc_refine_scan_read_workspace_bytes(int64_t batch, int64_t length, int64_t width, int64_t features);
int koemi_assoc_refine_scan_read(const void* projections, int projection_dtype, int64_t row_stride,
                                 int64_t value_offset, int64_t feature_offset, int64_t query_feature_offset,
                                 int64_t decay_offset, int64_t write_offset, const float* surprise,
                                 const uint8_t* valid, const float* novelty, float refine_decay_rate,
                                 const void* fast_read, int fast_dtype, int64_t fast_row_stride, const float* basis,
                                 const float* normalizer, void* read, int read_dtype, int64_t read_row_stride,
                                 float* next_basis, float* next_normalizer, int64_t batch, int64_t length,
                                 int64_t width, int64_t features, void* workspace, size_t workspace_bytes,
                                 koemi_stream_t stream);

/* koemi_assoc_refine_scan_read over a sequence of windows, as
 * koemi_assoc_scan_read_windows runs the fast memory (every window's terms,
 * the carried refine state of each window, every window's reads). */
size_t koemi_assoc_refine_scan_read_windows_workspace_bytes(int64_t batch, int64_t windows, int64_t window,
                                                            int64_t width, int64_t features);
int koemi_assoc_refine_scan_read_windows(const void* projections, int projection_dtype, int64_t row_stride,
                                         int64_t value_offset, int64_t feature_offset, int64_t query_feature_offset,
                                         int64_t decay_offset, int64_t write_offset, const float* surprise,
                                         const uint8_t* valid, const float* novelty, float refine_decay_rate,
                                         const void* fast_read, int fast_dtype, int64_t fast_row_stride,
                                         const float* basis, const float* normalizer, void* read, int read_dtype,
                                         int64_t read_row_stride, float* next_basis, float* next_normalizer,
                                         int64_t batch, int64_t windows, int64_t window, int64_t width,
                                         int64_t features, void* workspace, size_t workspace_bytes,
                                         koemi_stream_t stream);

/* Novelty output of LocalKeyValueMemory.read_window (model/memory.py:354-361)
 * for `rows` window rows of `length` queries: over the slots of [carried
 * (capacity) ; window (length)] eligible for query t (valid and among the
 * `window` positions strictly before its own, memory.py:364-383), the largest
 * cosine similarity k . q / (max(|k|, 1e-12) max(|q|, 1e-12)); novelty =
 * clamp(1 - largest, 0, 1), 1 without an eligible slot. carried_keys [rows,
 * capacity, width] fp32 with carried_valid [rows, capacity]; keys [rows,
 * length, width] (F32 or BF16, rows key_row_stride apart) with key_valid;
 * queries fp32 (rows query_row_stride apart); novelty [rows, length] fp32. */
int koemi_local_novelty(const float* carried_keys, const uint8_t* carried_valid, const void* keys, int key_dtype,
                        int64_t key_row_stride, const uint8_t* key_valid, const float* queries,
                        int64_t query_row_stride, float* novelty, int64_t rows, int64_t capacity, int64_t length,
                        int64_t width, int64_t window, koemi_stream_t stream);

/* The refine gate (KoemiModel.refine_memory, model/network.py:714-721): per
 * position, pre = W [working; fast; refine; local] + b (weight [4 width], bias
 * [1] fp32), g = sigmoid(pre), out = fast + g refine. round_bf16 != 0 (a bf16
 * stack: nn.Linear under bf16 autocast) rounds every input and the weight to
 * bf16 (weight BF16) and the pre-activation to bf16 after the bias; otherwise
 * every tensor is F32. working, fast and refine fp32; local F32 or BF16; out
 * F32 or BF16; every row stride 0 means width. */
int koemi_herm_refine_gate(const float* working, int64_t working_row_stride, const float* fast,
                           int64_t fast_row_stride, const float* refine, int64_t refine_row_stride, const void* local,
                           int local_dtype, int64_t local_row_stride, const void* weight, int weight_dtype,
                           const float* bias, int round_bf16, void* out, int out_dtype, int64_t out_row_stride,
                           int64_t rows, int64_t width, koemi_stream_t stream);

/* Small per-window steps of the HERM block (torch composites in the reference).
 * koemi_herm_rmsnorm: out = RootMeanSquareNorm(x + residual) * weight
 * (layers.py:14-16) on rows whose mask byte is set (all rows when mask is
 * NULL), out = x elsewhere (the expert mixture's valid-row select,
 * experts.py:134-136); x [rows, width] in input_dtype (KOEMI_F32 or
 * KOEMI_BF16), weight and out fp32, residual NULL or [rows, width] in
 * residual_dtype; width a multiple of 4, at most 2048;
 * `output_bf16` (NULL: none) receives a bf16 copy of out for a following
 * GEMM, and `output` may then be NULL.
 * koemi_herm_token_context: previous[b, t] = the last valid token before t
 * (carried_last[b] before the first), last[b] = the window's last valid token
 * or carried_last[b] (network.py:742-761); int64 ids, valid bytes. With
 * `valid` NULL the validity is ids != pad_id (network.py:303) and is written
 * to `valid_out`; `targets_out` (NULL: none) receives ids where valid and 0
 * elsewhere (the surprise targets, network.py:335). */
int koemi_herm_rmsnorm(const void* input, int input_dtype, const void* residual, int residual_dtype,
                       const float* weight, const uint8_t* mask, float* output, void* output_bf16, int64_t rows,
                       int64_t width, float eps, koemi_stream_t stream);
/* koemi_herm_rmsnorm of a split projection's result: the input is the sum,
 * in block order, of `parts` (1..8) fp32 blocks [rows, width] one after another
 * (koemi_linear_rows_split's partials), plus add_bias (fp32 [width] or
 * NULL), rounded to bf16 when round_bf16 != 0 (the projection's bf16 output
 * under autocast); no residual or mask. */
int koemi_herm_rmsnorm_parts(const float* parts_input, int parts, const float* add_bias, int round_bf16,
                             const float* weight, float* output, void* output_bf16, int64_t rows, int64_t width,
                             float eps, koemi_stream_t stream);
int koemi_herm_token_context(const int64_t* token_ids, const uint8_t* valid, const int64_t* carried_last,
                             int64_t* previous, int64_t* last, uint8_t* valid_out, int64_t* targets_out, int64_t pad_id,
                             int64_t batch, int64_t length, koemi_stream_t stream);

/* A greedy decode step's next tokens (TokenSampler with the greedy policy,
 * runtime/fast_decode.py:53-55, 82-84: argmax of the logits with the
 * padding id removed): ids[r] = the first column of maximal logits[r, :]
 * (rows row_stride apart, fp32 [rows, vocab]) with column exclude_id scored
 * -inf, a NaN counting as the maximum (torch.argmax's rule). */
int koemi_herm_greedy_tokens(const float* logits, int64_t row_stride, int64_t rows, int64_t vocab, int64_t exclude_id,
                             int64_t* ids, koemi_stream_t stream);

/* TokenSampler's non-greedy draw (runtime/fast_decode.py:57-95) for `rows`
 * rows of fp32 logits (rows row_stride apart; 0: vocab): the exclude_id
 * column (PAD) removed, with top_k > 0 every score below the min(top_k,
 * vocab)-th largest removed (ties kept), p = softmax(score / temperature),
 * ids[r] the first column whose cumulative p (column order) exceeds
 * uniforms[r] in [0, 1) (the last column with p > 0 when rounding leaves
 * none). probabilities (NULL: none) receives p [rows, vocab]. The caller
 * draws the uniforms; vocab <= 4096. */
int koemi_herm_sample_tokens(const float* logits, int64_t row_stride, int64_t rows, int64_t vocab,
                             int64_t exclude_id, float temperature, int64_t top_k, const float* uniforms,
                             int64_t* ids, float* probabilities, koemi_stream_t stream);

/* causal_surprise of a HERM window from the state before each position
 * (network.py:318-325, 677-698) with the fixed-threshold admission
 * (network.py:349), one kernel: row (b, t) of the batch x length rows is
 * scored, as koemi_surprise_rows_forward does (fp32, content_bias `bias`
 * [vocab] or NULL), on the logits of row (b, t - 1) of `logits`
 * [batch * length, vocab] (the window's own states), and for t == 0 on row b
 * of `first` [batch, vocab] (the carried state), against target_ids[b, t];
 * `admission` (NULL: none) receives valid && surprise > threshold.
 * vocab == 256; 16-byte aligned logits. */
int koemi_herm_surprise_shifted(const float* logits, const float* first, const float* bias, const int64_t* target_ids,
                                const uint8_t* valid_mask, float* surprise, uint8_t* admission, float threshold,
                                int64_t batch, int64_t length, int64_t vocab, float log_vocab, koemi_stream_t stream);

/* The surprise and admission of a decode step in every layer at once (each
 * layer's one position scored on its carried state's content logits,
 * network.py:318-325, 349, 677-698): row (l, b) of logits [layers * batch,
 * vocab] is scored with the content bias biases[l] (a host array of `layers`
 * fp32 [vocab] pointers, read during the call) against target_ids[b] and
 * valid_mask[b], into surprise[l * batch + b] and admission[l * batch + b]
 * (NULL: none); the arithmetic of koemi_herm_surprise_shifted at length 1.
 * layers <= 32, vocab == 256. */
int koemi_herm_surprise_layers(const float* logits, const float* const* biases, const int64_t* target_ids,
                               const uint8_t* valid_mask, float* surprise, uint8_t* admission, float threshold,
                               int layers, int64_t batch, int64_t vocab, float log_vocab, koemi_stream_t stream);

/* The fusion layer's input [working ; memory ; local ; salient]
 * (network.py:401-405, a torch.cat in the reference) as one bf16 matrix
 * [rows, pieces * width] for its GEMM: `pieces` (1..4) fp32 [rows, width]
 * blocks (16-byte aligned), width % 4 == 0, rounded to nearest even. */
int koemi_herm_concat_bf16(const float* input0, const float* input1, const float* input2, const float* input3,
                           int pieces, int64_t rows, int64_t width, void* output, koemi_stream_t stream);

/* Local-memory read, LocalKeyValueMemory.read_window of model/memory.py:332-362
 * without the novelty output (a torch composite in the reference; network.py:
 * 328-336). The read of koemi_salient_read with the sliding window of
 * memory.py:364-383: slot s (carried entries, then the window's entries) is
 * eligible for query t when its valid byte (carried_valid, then valid) is set
 * and carried + t - window <= s < carried + t. Same layouts, dtypes and
 * workspace (koemi_salient_read_workspace_bytes) as koemi_salient_read;
 * window >= 1. */
int koemi_local_read(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                     const void* keys, const void* values, const uint8_t* valid, const void* queries, void* out,
                     int64_t batch, int64_t carried, int64_t length, int64_t width, int64_t window, int dtype,
                     void* workspace, size_t workspace_bytes, koemi_stream_t stream);

/* The salient (window = 0) or local (window >= 1) read of koemi_salient_read /
 * koemi_local_read, fp32 inputs, written as out_dtype (KOEMI_F32 or
 * KOEMI_BF16) rows `out_row_stride` elements apart, so that the read can land
 * in a column block of a wider matrix (the HERM fusion layer's bf16 input,
 * network.py:401-405, without a separate concatenation). Only the one-launch
 * fused read: width % 8 == 0, 16-byte aligned fp32 rows, at most 152
 * candidate slots per 32 queries (salient: carried + length - 1 <= 152;
 * local: carried <= 64 and window <= 33); other shapes return
 * KOEMI_ERR_UNSUPPORTED (take koemi_salient_read / koemi_local_read). No
 * workspace. The window's keys and values are rows key_row_stride elements
 * apart (0: width, else a multiple of 4; of 8 for bf16) of key_dtype
 * KOEMI_F32 or KOEMI_BF16 (the bf16 columns of the block's key/value
 * projection read in place, widened exactly; keys 16-byte aligned). Every slot a query can see is
 * flagged valid, so masking the window's invalid entries changes nothing. */
int koemi_memory_read_into(const float* carried_keys, const float* carried_values, const uint8_t* carried_valid,
                           const void* keys, const void* values, int key_dtype, int64_t key_row_stride,
                           const uint8_t* flags, const float* queries, void* out, int out_dtype,
                           int64_t out_row_stride, int64_t batch, int64_t carried, int64_t length, int64_t width,
                           int64_t window, koemi_stream_t stream);

/* Replaces `combine_topk(y, rows, offsets, T, k)` of moe/moe_kernels.cu:560-582
 * without atomics: combined[t] = sum over the valid sorted pairs i of token t,
 * in ascending i, of y_i * w_i in fp32, w_i = pair_weights[i] (sorted order)
 * or 1/top_k when pair_weights is NULL; tokens without pairs get 0. Output in
 * `dtype` (the expert_outputs dtype). num_segments = len(segment_offsets) - 1. */
size_t koemi_moe_combine_workspace_bytes(int64_t tokens, int64_t top_k);
int koemi_moe_combine(const void* expert_outputs, const int64_t* sorted_rows,
                      const int64_t* segment_offsets, const float* pair_weights, void* combined,
                      int64_t pairs, int64_t width, int64_t tokens, int64_t top_k,
                      int64_t num_segments, int dtype, void* workspace, size_t workspace_bytes,
                      koemi_stream_t stream);

/* The HERM block's expert tail in one pass (no single reference op): the
 * combine of koemi_moe_combine (bf16 expert outputs [pairs, width], the
 * ascending-position fp32 sum of each token's pairs scaled by pair_weights or
 * 1/top_k, rounded once to bf16: combine_topk, moe/__init__.py), the expert
 * output normalizer RMSNorm(context + update) * expert_norm_weight with rows
 * whose mask is false keeping the context (experts.py:134-136,
 * layers.py:14-16), and, with next_norm_weight, the next block's input
 * RMSNorm of that result (network.py:296-310). Each step rounds as the
 * separate kernels do (koemi_moe_combine, then koemi_herm_rmsnorm twice), so
 * the outputs are the same bits. context [tokens, width] fp32; output (NULL:
 * none) [tokens, width] fp32; next_input_bf16 (NULL: none) [tokens, width]
 * bf16. top_k <= 8, width % 4 == 0 and <= 2048, 16-byte aligned rows. The
 * pairs of each token come from pair_positions when given (the permutation's
 * pair -> sorted position map of koemi_moe_permute_indices; no workspace),
 * else from inverting sorted_rows (the workspace of
 * koemi_moe_combine_workspace_bytes(tokens, top_k)). */
int koemi_herm_combine_norm(const void* expert_outputs, const int64_t* sorted_rows, const int64_t* pair_positions,
                            const int64_t* segment_offsets, const float* pair_weights, const float* context,
                            const uint8_t* mask,
                            const float* expert_norm_weight, const float* next_norm_weight, float* output,
                            void* next_input_bf16, int64_t pairs, int64_t width, int64_t tokens, int64_t top_k,
                            int64_t num_segments, float eps, void* workspace, size_t workspace_bytes,
                            koemi_stream_t stream);

/* koemi_herm_combine_norm with the context formed in place (no reference
 * counterpart; a build-side fusion of the HERM block's tail): the context is
 * the fusion normalizer's output RMSNorm(fusion_rows) * fusion_norm_weight
 * (network.py:723-732) of the bf16 fusion rows [tokens, width] (the fusion
 * layer's output, bias included), with the arithmetic of koemi_herm_rmsnorm
 * on those rows, so the outputs equal koemi_herm_rmsnorm followed by
 * koemi_herm_combine_norm on its fp32 result bit for bit, and the fp32
 * context never goes through memory. Pairs by pair_positions only; the
 * other arguments as koemi_herm_combine_norm. */
int koemi_herm_combine_norm_fusion(const void* expert_outputs, const int64_t* pair_positions,
                                   const int64_t* segment_offsets, const float* pair_weights,
                                   const void* fusion_rows, const float* fusion_norm_weight, const uint8_t* mask,
                                   const float* expert_norm_weight, const float* next_norm_weight, float* output,
                                   void* next_input_bf16, int64_t pairs, int64_t width, int64_t tokens,
                                   int64_t top_k, int64_t num_segments, float eps, koemi_stream_t stream);

/* Measurement only (no counterpart in the reference): reads `bytes` (a
 * multiple of 16) from `src` with `grid` workgroups of `block` threads, each
 * thread issuing `unroll` (1, 2, 4 or 8) 16-byte loads per pass of a
 * grid-stride loop; `sink` (grid * block floats) is written only for a sum
 * the benchmark never produces. bench.py --read-floor sweeps the launch shape
 * to find the fastest plain read of a given size on the chip, the floor the
 * memory-bound kernels are judged against. */
int koemi_stream_read(const void* src, int64_t bytes, int unroll, int block, int64_t grid, float* sink,
                      koemi_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KOEMI_HIP_H */
