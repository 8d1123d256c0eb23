/* sparsebench_hip.h: C ABI of the MI355X (gfx950) MoE forward path.
 *
 * One shared library, libsparsebench_hip.so, built by hipcc for gfx950 only.
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (passed as void*, so a binder needs no HIP headers), enqueues work on that
 * stream and returns at once: no allocation, no host sync, no hipMalloc, so
 * every call may be recorded into a HIP graph. Buffers are owned by the
 * caller. Return value: SB_OK, or an SB_ERR_* code with a message readable
 * through sb_last_error() on the calling thread.
 *
 * Each entry point names the reference interface it replaces, in
 * saransh-debugs/SparseBench (paths relative to that repository).
 */
#ifndef SPARSEBENCH_HIP_H_
#define SPARSEBENCH_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SB_OK 0
#define SB_ERR_INVALID 1 /* bad argument: shape, size, alignment, range */
#define SB_ERR_HIP 2     /* a HIP runtime call or kernel launch failed */

/* Element type codes for sb_combine's gate weights. */
#define SB_DTYPE_BF16 0
#define SB_DTYPE_F16 1
#define SB_DTYPE_F32 2

/* Message of the last failed call on this thread ("" if none). */
const char* sb_last_error(void);

/* Library version, for a binder to check it loaded the right file. */
int32_t sb_version(void);

/* No counterpart in the reference: test hooks, process-wide overrides of a
 * choice the library otherwise makes itself (value 0 restores the choice).
 * For tests that must reach each code path; outputs do not depend on them.
 *   SB_HOOK_EXPERT_GATE  1: the layer kernels' expert tiles, 2: row blocks
 *   SB_HOOK_TOPK_KERNEL  1: the top-k router's wave form, 2: its lane form */
#define SB_HOOK_EXPERT_GATE 0
#define SB_HOOK_TOPK_KERNEL 1
#define SB_NUM_TEST_HOOKS 2
int sb_set_test_hook(int32_t hook, int32_t value);

/* Replaces arch_probe (csrc/smoke.cu:23-38, csrc/ops.hpp:11).
 * Writes the architecture number of the code that ran (950 on gfx950)
 * into out[0..n). n must be positive. */
int sb_arch_probe(int32_t* out, int64_t n, void* stream);

/* Worst-case sizes of the routing outputs for n = T*k copies
 * (csrc/routing.cu:213-216). Host-only arithmetic; returns SB_ERR_INVALID
 * when the problem does not fit int32 indexing. */
int sb_routing_sizes(int64_t num_copies, int32_t num_experts, int32_t ffn_dim, int32_t block_size,
                     int64_t* max_row_blocks, int64_t* max_rows, int64_t* workspace_elems);

/* Replaces build_topology_cuda (csrc/routing.cu:197-281, csrc/ops.hpp:20-21).
 * expert_idx: [T, k] int32 (idx_is_i64 = 0) or int64 (idx_is_i64 = 1).
 * Writes, for the worst-case sizes given by sb_routing_sizes:
 *   tokens_per_expert[E], padded_offsets[E+1], row_token[max_rows],
 *   copy_row[T*k], row_block_expert[max_row_blocks],
 *   row_offsets[max_row_blocks+1], col_indices[max_row_blocks*ffn_blocks],
 *   error[1] (1 if any expert id was outside [0, E), else 0).
 * workspace: workspace_elems int32 of scratch, owned by the caller.
 * valid_tokens: NULL for the reference behaviour; otherwise a device int32
 * holding T' <= T, and copies of tokens >= T' are neither counted nor
 * flagged (copy_row = -1): a graph captured at T can replay at T' <= T.
 * Outputs are bit-identical to sparsebench/topology.py:build_topology on the
 * live part, with the past-the-end conventions of routing.cu:162-193, 248-249. */
int sb_routing(const void* expert_idx, int32_t idx_is_i64, int64_t num_tokens, int32_t k, int32_t num_experts,
               int32_t ffn_dim, int32_t block_size, const int32_t* valid_tokens, int32_t* workspace,
               int32_t* tokens_per_expert, int32_t* padded_offsets, int32_t* row_token, int32_t* copy_row,
               int32_t* row_block_expert, int32_t* row_offsets, int32_t* col_indices, int32_t* error, void* stream);

/* No counterpart in the reference: sb_routing for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same arguments and outputs as sb_routing, without
 * `workspace`: the per-chunk counts live in a fixed device array of
 * 524288 int32 (2 MiB) that each GPU holds until the process ends. Problems
 * that need more scratch (ceil(T*k / 1024) * (E + 1) int32, from
 * sb_routing_sizes) are rejected with SB_ERR_INVALID. The array used is
 * that of the stream's device (the current device for the null stream);
 * the first call on a device looks it up (make it outside graph capture);
 * no call allocates. Calls that overlap on one GPU share the array and
 * race: issue them on one stream. */
int sb_routing_noalloc(const void* expert_idx, int32_t idx_is_i64, int64_t num_tokens, int32_t k,
                       int32_t num_experts, int32_t ffn_dim, int32_t block_size, const int32_t* valid_tokens,
                       int32_t* tokens_per_expert, int32_t* padded_offsets, int32_t* row_token, int32_t* copy_row,
                       int32_t* row_block_expert, int32_t* row_offsets, int32_t* col_indices, int32_t* error,
                       void* stream);

/* Replaces sdd_cuda (csrc/sdd.cu:123-170, csrc/ops.hpp:34-36).
 * out[num_row_blocks*F/128, 128, 128] bf16 = (gelu)(x[row_token] @ w1[expert])
 * on the layout's blocks. x [T, D] bf16, w1 [E, D, F] bf16, 16-byte aligned;
 * D % 64 == 0, F % 256 == 0; row_token has num_row_blocks*128 entries.
 * Rows with row_token < 0 are zero (no read of x); row blocks with
 * row_offsets[r] == row_offsets[r+1] are skipped and their blocks left unwritten.
 * gelu is the erf form in fp32 (erfc to 1.5e-7, Abramowitz & Stegun 7.1.26),
 * then round to nearest even; gelu(+-0) = +0, gelu(+inf) = +inf, NaN stays
 * NaN, and gelu(-inf) = 0 where the erf formula gives NaN. */
int sb_sdd(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
           const int32_t* row_offsets, void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim,
           int64_t num_experts, int64_t num_row_blocks, int32_t apply_gelu, void* stream);

/* Replaces dsd_cuda's kernels (csrc/dsd.cpp:27-80, csrc/dsd_v5.cu:106-123,
 * csrc/ops.hpp:27-28).
 * out[num_row_blocks*bs, D] bf16 = BSR(blocks, row_offsets, col_indices) @ w.
 * blocks [nnz, bs, bs] bf16, w [w_rows, D] bf16, bs in {64, 128}, D % 128 == 0.
 * zero_dead_rows = 1 writes zeros for row blocks with no blocks (the contract
 * of versions 1-3); 0 leaves them unwritten (versions 4, 41, 5). */
int sb_dsd(const void* blocks, const void* w, const int32_t* row_offsets, const int32_t* col_indices, void* out,
           int64_t nnz, int64_t w_rows, int64_t num_row_blocks, int64_t block_size, int64_t d_model,
           int32_t zero_dead_rows, void* stream);

/* Replace the SDD and DSD stages of moe_forward (sparsebench/moe.py:46-48:
 * spmm.sdd then spmm.dsd version 5 on route_device's layout). Each call
 * enqueues one kernel whose workgroups choose, on the GPU and all alike from
 * tokens_per_expert, between tiles that follow each expert's real rows and
 * row-block tiles of sb_sdd's / sb_dsd's default shape. The DSD's expert
 * tiles run when no expert holds more than twice the mean rows, F >= 1536
 * and the DSD's grid holds them; the SDD's run when the DSD's do and either the
 * experts hold at most 256 rows on average or the expert tiles need fewer
 * rounds over the device's CUs than the row blocks. An expert's weights
 * are then streamed once per chunk of up to 192 rows (SDD) or 256 rows
 * (DSD; 320 when F >= 8192, a last piece of up to 64 rows joining the
 * chunk before it) instead of once per row block, and padding rows past
 * the last 32-row group are neither computed nor read. For F % 512 != 0
 * sb_sdd_experts tiles each expert's row blocks in pairs (256 x 256 tiles,
 * an odd last one alone) and writes every padded row, as sb_sdd does,
 * except, when F < 8192, rows past the first 64 of an expert of at most 64
 * rows (the DSD's row-block tiles do not read them). It
 * calls sb_sdd itself when x or one expert's W1 is 2 GiB or more (the layer
 * kernels address them with 32-bit offsets).
 * The layout arrays are sb_routing's outputs (or those of
 * sb_routing_assigned / sb_token_rounding); max_row_blocks is its
 * worst-case row block count and num_copies the length of its copy_row.
 * Every real row of out equals, bit for bit, what sb_sdd / sb_dsd write for
 * it. sb_sdd_experts writes zeros on the padding rows up to each expert's
 * next multiple of 32 rows; other padding rows may be left unwritten, as
 * may every padding row of sb_dsd_experts's out[max_row_blocks*128, D].
 * SDD: D % 64 == 0, F % 256 == 0. DSD: F % 128 == 0, D % 256 == 0, and h
 * (max_row_blocks*F/128 blocks) under 2 GB. */
int sb_sdd_experts(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
                   const int32_t* row_offsets, const int32_t* tokens_per_expert, const int32_t* padded_offsets,
                   void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim, int64_t num_experts,
                   int64_t max_row_blocks, int32_t apply_gelu, void* stream);
int sb_dsd_experts(const void* h, const void* w2, const int32_t* tokens_per_expert, const int32_t* padded_offsets,
                   const int32_t* row_block_expert, const int32_t* row_offsets, const int32_t* col_indices, void* out,
                   int64_t max_row_blocks, int64_t num_experts, int64_t num_copies, int64_t ffn_dim, int64_t d_model,
                   void* stream);

/* Replaces the combine step of moe_forward (sparsebench/moe.py:51-54).
 * out[t, :] = bf16( sum_j fp32(y[copy_row[t*k+j], :]) * fp32(gates[t*k+j]) ),
 * j in [0, k), fp32 accumulation. Copies with copy_row < 0 add nothing.
 * y [y_rows, D] bf16, out [T, D] bf16, gates [T, k] of gate_dtype, D % 8 == 0.
 * valid_tokens: NULL, or a device int32 T' <= T: rows t >= T' are not written. */
int sb_combine(const void* y, const int32_t* copy_row, const void* gates, int32_t gate_dtype, void* out,
               int64_t num_tokens, int32_t k, int64_t d_model, int64_t y_rows, const int32_t* valid_tokens,
               void* stream);

/* ---- Routing given as assignments (sparsebench/moe.py:59-91) ---------- */

/* Replaces the routing of moe_forward_assigned (sparsebench/moe.py:80-84:
 * route_device on expert_of_copy as [N, 1], then row_token remapped from
 * copy index to token). Copy c sends token_of_copy[c] (int32/int64) to
 * expert_of_copy[c] (int32/int64). The outputs are those of sb_routing with
 * T*k replaced by N = num_copies and row_token holding token ids; size them
 * with sb_routing_sizes(N, ...). A token id outside [0, num_tokens) is
 * treated like a bad expert id (copy skipped, error = 1); the reference
 * would index out of range there. valid_tokens: as for sb_routing, with the
 * copy's token id compared to T'. */
int sb_routing_assigned(const void* expert_of_copy, int32_t expert_is_i64, const void* token_of_copy,
                        int32_t token_is_i64, int64_t num_copies, int64_t num_tokens, int32_t num_experts,
                        int32_t ffn_dim, int32_t block_size, const int32_t* valid_tokens, int32_t* workspace,
                        int32_t* tokens_per_expert, int32_t* padded_offsets, int32_t* row_token, int32_t* copy_row,
                        int32_t* row_block_expert, int32_t* row_offsets, int32_t* col_indices, int32_t* error,
                        void* stream);

/* Each token's copies, for the assigned combine (the grouping that the
 * reference leaves to index_add_ at sparsebench/moe.py:89-91). Writes
 * token_offsets[T+1] and token_copies[N]: the copies of token t are
 * token_copies[token_offsets[t] .. token_offsets[t+1]), in ascending copy
 * order; copies with copy_row < 0 are left out and the unused tail of
 * token_copies is -1. One workgroup; deterministic. */
int sb_token_csr(const void* token_of_copy, int32_t token_is_i64, const int32_t* copy_row, int64_t num_copies,
                 int64_t num_tokens, int32_t* token_offsets, int32_t* token_copies, void* stream);

/* Replaces the combine of moe_forward_assigned (sparsebench/moe.py:89-91).
 * out[t, :] = bf16( sum over t's copies c, in token_copies order, of
 * fp32(y[copy_row[c], :]) * fp32(weights[c]) ); zeros for a token with no
 * copy. token_copies may be NULL when the copies are already in token order
 * (then copy i of the range is c = i). weights [N] of weight_dtype.
 * valid_tokens: NULL, or a device int32 T' <= T: rows t >= T' not written. */
int sb_combine_assigned(const void* y, const int32_t* copy_row, const void* weights, int32_t weight_dtype,
                        const int32_t* token_offsets, const int32_t* token_copies, void* out, int64_t num_tokens,
                        int64_t d_model, int64_t y_rows, const int32_t* valid_tokens, void* stream);

/* ---- Router: top-k and token rounding (sparsebench/token_rounding.py) -- */

/* Sizes for token rounding of scores [T, E] at top-k with the given tile,
 * and the layout (block_size, ffn_dim) built from it: the list capacity
 * (N <= min(T*E, T*k + E*(tile/2)): an expert moves up by less than half a
 * tile), the layout's worst-case row blocks / rows (sb_routing_sizes of the
 * capacity) and the int32 workspace of sb_token_rounding. Host-only. */
int sb_router_sizes(int64_t num_tokens, int32_t num_experts, int32_t k, int32_t tile, int32_t block_size,
                    int32_t ffn_dim, int64_t* max_assignments, int64_t* max_row_blocks, int64_t* max_rows,
                    int64_t* workspace_elems);

/* Replaces top_k_assignments (sparsebench/token_rounding.py:39-46):
 * scores [T, E] fp32 -> top_idx [T, k] int32, the k best experts of each
 * token in descending score order (equal scores: lower expert first), and
 * top_weight [T, k] fp32 = the picked scores over their sum. k <= 16. */
int sb_router_topk(const float* scores, int64_t num_tokens, int32_t num_experts, int32_t k, int32_t* top_idx,
                   float* top_weight, void* stream);

/* Replaces token_rounding (sparsebench/token_rounding.py:58-81), fused with
 * the routing of moe_forward_assigned, with no host sync.
 * scores [T, E] fp32. Writes the rounded routing as a list in (token,
 * expert) order, capacity max_assignments (sb_router_sizes):
 *   token_of_copy, expert_of_copy (int32), weight_of_copy (fp32), entries
 *   past the real length -1 / -1 / 0; num_assignments[1] = the length N;
 *   token_offsets[T+1]: token t's copies are token_offsets[t] .. [t+1]
 *   (pass NULL token_copies to sb_combine_assigned);
 * and its block-sparse layout, as sb_routing_assigned would build it from
 * that list (tokens_per_expert = the rounded counts; copy_row[capacity]).
 * workspace: workspace_elems int32 (sb_router_sizes). E <= 1024, k <= 16. */
int sb_token_rounding(const float* scores, int64_t num_tokens, int32_t num_experts, int32_t k, int32_t tile,
                      int32_t block_size, int32_t ffn_dim, int32_t* workspace, int32_t* token_of_copy,
                      int32_t* expert_of_copy, float* weight_of_copy, int32_t* num_assignments,
                      int32_t* token_offsets, int32_t* tokens_per_expert, int32_t* padded_offsets,
                      int32_t* row_token, int32_t* copy_row, int32_t* row_block_expert, int32_t* row_offsets,
                      int32_t* col_indices, int32_t* error, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARSEBENCH_HIP_H_ */
