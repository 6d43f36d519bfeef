/*
 * semblend_hip.h — C ABI of libsemblend_hip.so, the MI355X (gfx950) kernel library
 * behind SemBlend's KV-reuse path: donor-KV scatter into a paged cache, RoPE delta
 * correction of donor K, and partial-prefill attention.
 *
 * Conventions shared by every entry point
 *   - All tensor arguments are device pointers owned by the caller. The library never
 *     allocates: any workspace is passed in by the caller, sized as documented.
 *   - Strides are in ELEMENTS (not bytes) and are passed as host arrays of int64_t, so the
 *     standard [num_blocks, 2, heads, block_size, head_dim] cache, vLLM's flash-attn
 *     [2, num_blocks, block_size, heads, head_dim] cache and TRT-LLM's
 *     [num_blocks, 2, block_size, heads, head_dim] cache are all addressed without copies.
 *   - Index arrays (positions, block tables) are int32 device arrays.
 *   - dtype is one of SB_DTYPE_*; RoPE and attention arithmetic is fp32.
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream); work is
 *     enqueued asynchronously and the call never synchronises the device.
 *   - Return value: SB_OK (0), SB_ERR_INVALID_ARGUMENT, or a hipError_t value from the
 *     launch. sb_last_error_string() describes the last failure on the calling thread.
 *   - Out-of-range pairs (donor position >= donor length, logical block beyond the block
 *     table, physical block >= pool size, negative positions) are skipped silently, as the
 *     reference's GPU kernels skip them.
 */
#ifndef SEMBLEND_HIP_H
#define SEMBLEND_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SB_OK 0
#define SB_ERR_INVALID_ARGUMENT 100001

#define SB_DTYPE_F32 0
#define SB_DTYPE_F16 1
#define SB_DTYPE_BF16 2

/* Flags of the multi-layer scatters (sb_*_paged_layers, sb_composite_scatter_paged_layers).
 * SB_SCATTER_REPEATED_DONOR_ROWS: a donor row may be the source of several pairs (one
 * donor position mapped to several targets). The launch then reads the donor through the
 * caches so that the repeats are served from L2 / Infinity Cache; without it the donor is
 * read with nontemporal loads, which is faster when every donor row is read once. Either
 * setting gives the same results. */
#define SB_SCATTER_REPEATED_DONOR_ROWS 1
#define SB_SCATTER_FLAGS_ALL 1

/* Most positions sb_apply_rope_delta_inplace_host takes (they travel inside the launch). */
#define SB_INLINE_POSITIONS_MAX 256

/* Library version string, e.g. "semblend_hip 0.1.0 gfx950". */
const char* sb_version(void);

/* Description of the last failure on the calling thread ("" if none). */
const char* sb_last_error_string(void);

/* ------------------------------------------------------------------------------------------
 * Donor-KV scatter
 * ---------------------------------------------------------------------------------------- */

/* Flat scatter over all layers:
 *   target[l, kv, h, t, :] = donor[l, kv, h, d, :] for every pair (d, t).
 * target [L, 2, H, St, D] with strides t_strides[5]; donor [L, 2, H, Sd, D] with d_strides[5].
 * Replaces semblend_core/triton_kernels.py:132-191 (scatter_donor_kv, kernel :59-129). */
int sb_scatter_donor_kv(void* target, const void* donor, const int32_t* donor_pos,
                        const int32_t* target_pos, int64_t num_pairs, int64_t num_layers,
                        int64_t num_heads, int64_t head_dim, int64_t target_seq_len,
                        int64_t donor_seq_len, const int64_t* t_strides,
                        const int64_t* d_strides, int32_t dtype, void* stream);

/* Paged scatter, one layer:
 *   kv_cache[bt[t / bs], kv, h, t % bs, :] = donor_kv[kv, h, d, :].
 * kv_cache [NB, 2, H, bs, D] addressed by kv_strides[5] = (block, kv, head, pos, dim);
 * donor_kv [2, H, Sd, D] addressed by d_strides[4].
 * Replaces semblend_core/triton_kernels.py:279-356 (scatter_donor_kv_paged, kernel :200-276). */
int sb_scatter_donor_kv_paged(void* kv_cache, const void* donor_kv, const int32_t* block_table,
                              const int32_t* donor_pos, const int32_t* target_pos,
                              int64_t num_pairs, int64_t num_heads, int64_t block_size,
                              int64_t head_dim, int64_t donor_seq_len, int64_t num_blocks_total,
                              int64_t num_blocks_per_seq, const int64_t* kv_strides,
                              const int64_t* d_strides, int32_t dtype, void* stream);

/* Paged scatter over several layers in one launch. kv_layer_ptrs / donor_layer_ptrs are
 * DEVICE arrays of num_layers base addresses (uint64); every layer shares the strides.
 * flags: 0 or SB_SCATTER_REPEATED_DONOR_ROWS (other bits are rejected).
 * No reference counterpart: it replaces the per-layer loop of callers such as
 * synapse_kv_connector/model_runner_hook.py:215-276. */
int sb_scatter_donor_kv_paged_layers(const uint64_t* kv_layer_ptrs,
                                     const uint64_t* donor_layer_ptrs, int64_t num_layers,
                                     const int32_t* block_table, const int32_t* donor_pos,
                                     const int32_t* target_pos, int64_t num_pairs,
                                     int64_t num_heads, int64_t block_size, int64_t head_dim,
                                     int64_t donor_seq_len, int64_t num_blocks_total,
                                     int64_t num_blocks_per_seq, const int64_t* kv_strides,
                                     const int64_t* d_strides, int32_t dtype, int32_t flags,
                                     void* stream);

/* ------------------------------------------------------------------------------------------
 * QKV projection (bf16 / fp16 on the matrix cores, fp32 accumulation, one rounding)
 * ---------------------------------------------------------------------------------------- */

/* Masked QKV projection as a compacted GEMM:
 *   out[s, :] = hidden[s, :] W^T + bias   where compute_mask[s] != 0, 0 elsewhere.
 * hidden [seq_len, hidden_dim] (row stride hidden_stride), W [out_features, hidden_dim]
 * (row stride weight_stride), bias [out_features] in the same dtype or NULL, out
 * [seq_len, out_features] (row stride out_stride); strides in elements. The mask is
 * compacted on the device into `workspace` (sb_masked_qkv_projection_workspace_size bytes),
 * and only the computed rows are multiplied. hidden_dim must be a multiple of 64,
 * out_features of 8, all rows 16-byte aligned.
 * Replaces semblend_core/triton_kernels.py:451-522 for bf16 / fp16. */
int64_t sb_masked_qkv_projection_workspace_size(int64_t seq_len);
int sb_masked_qkv_projection(void* out, const void* hidden, const void* weight, const void* bias,
                             const uint8_t* compute_mask, void* workspace,
                             int64_t workspace_bytes, int64_t seq_len, int64_t hidden_dim,
                             int64_t out_features, int64_t hidden_stride, int64_t weight_stride,
                             int64_t out_stride, int32_t dtype, void* stream);

/* Compacted GQA QKV projection fused with the new K/V write: for each row n the hidden row
 * p = positions[n] is projected with W [(Hq + 2 Hkv) * D, hidden_dim] (+ bias), features
 * laid out Q | K | V. With inv_freq (device fp32 [D/2]), Q and K are rotated by p with the
 * interleaved RoPE (angle p * inv_freq[i]) before the rounding. Q goes to q_out[n]
 * ([num_rows, Hq * D], row stride q_stride); K and V go to the paged cache slot of p
 * (kv_strides[5] = block, kv, head, pos, dim in elements), skipped when the slot is out of
 * range. A row whose position is outside [0, seq_len) gets a zero Q row and writes no K/V.
 * head_dim must be a multiple of 8 and every row (hidden, W, q_out, cache) 16-byte aligned.
 * `workspace` (16-byte aligned, sb_qkv_projection_paged_workspace_size bytes) holds the
 * per-row cos/sin table with RoPE and, for row counts too small to give every CU a tile,
 * the fp32 partial products of a split of the hidden dimension (summed in a fixed order by
 * the epilogue); it may be NULL when that size is 0.
 * No reference counterpart: it fuses masked_qkv_projection (triton_kernels.py:451-522) with
 * the K/V write of partial_prefill (:904-909) into the paged layout, for GQA models. */
int64_t sb_qkv_projection_paged_workspace_size(int64_t num_rows, int64_t num_q_heads,
                                               int64_t num_kv_heads, int64_t head_dim,
                                               int64_t hidden_dim, int32_t rope);
int sb_qkv_projection_paged(void* q_out, const void* hidden, const void* weight,
                            const void* bias, const int32_t* positions, int64_t num_rows,
                            int64_t seq_len, int64_t hidden_dim, int64_t num_q_heads,
                            int64_t num_kv_heads, int64_t head_dim, const float* inv_freq,
                            void* workspace, int64_t workspace_bytes, void* kv_cache, const int32_t* block_table, int64_t block_size,
                            int64_t num_blocks_total, int64_t num_blocks_per_seq,
                            int64_t hidden_stride, int64_t weight_stride, int64_t q_stride,
                            const int64_t* kv_strides, int32_t dtype, void* stream);

/* Library-GEMM form of sb_qkv_projection_paged, in three steps around a GEMM the caller
 * runs (hipBLASLt): sb_qkv_gather_rows copies hidden row positions[n] to xg[n] ([num_rows,
 * hidden_dim] contiguous; rows without a valid position are zero) and, with inv_freq,
 * fills rope_table (num_rows * head_dim * 4 bytes, as the workspace of
 * sb_qkv_projection_paged) in the same launch; the caller computes proj = xg . W^T in fp32;
 * sb_qkv_epilogue_paged adds the bias, rotates Q and K by the row's position from
 * rope_table (NULL: no RoPE), rounds once to dtype and writes Q to q_out (compact) and K / V
 * into the paged cache: the same results as the fused kernel on the same products. Rows
 * whose position is outside [0, seq_len) get a zero Q row and no K / V write.
 * Fuse the K/V write of semblend_core/triton_kernels.py:904-909 and the RoPE at the new
 * positions into the GEMM's epilogue; no reference counterpart. */
int sb_qkv_gather_rows(void* xg, const void* hidden, const int32_t* positions,
                       int64_t num_rows, int64_t seq_len, int64_t hidden_dim,
                       int64_t hidden_stride, const float* inv_freq, int64_t head_dim,
                       void* rope_table, int32_t dtype, void* stream);
int sb_qkv_epilogue_paged(void* q_out, const float* proj, const void* bias,
                          const int32_t* positions, int64_t num_rows, int64_t seq_len,
                          int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                          const void* rope_table, void* kv_cache, const int32_t* block_table,
                          int64_t block_size, int64_t num_blocks_total,
                          int64_t num_blocks_per_seq, int64_t proj_stride, int64_t q_stride,
                          const int64_t* kv_strides, int32_t dtype, void* stream);

/* ------------------------------------------------------------------------------------------
 * RoPE delta correction (interleaved pairs (2i, 2i+1); inv_freq is a device fp32 array of
 * head_dim/2 entries, 1 / base^(2i/head_dim))
 * ---------------------------------------------------------------------------------------- */

/* Fused scatter + RoPE: V copied; K rotated by (t - d) and rounded once to the cache dtype.
 * Same arguments as sb_scatter_donor_kv_paged plus inv_freq.
 * Replaces semblend_core/rope_correction.py:193-282 (kernel :66-190, CPU path :285-328). */
int sb_rope_correct_scatter_paged(void* kv_cache, const void* donor_kv,
                                  const int32_t* block_table, const int32_t* donor_pos,
                                  const int32_t* target_pos, const float* inv_freq,
                                  int64_t num_pairs, int64_t num_heads, int64_t block_size,
                                  int64_t head_dim, int64_t donor_seq_len,
                                  int64_t num_blocks_total, int64_t num_blocks_per_seq,
                                  const int64_t* kv_strides, const int64_t* d_strides,
                                  int32_t dtype, void* stream);

/* Multi-layer form of sb_rope_correct_scatter_paged (device arrays of layer base addresses
 * and flags as in sb_scatter_donor_kv_paged_layers). cos/sin are computed once per pair and
 * shared by every layer and head. No reference counterpart (replaces a per-layer caller loop, e.g.
 * semblend/integration/trtllm/pytorch_backend.py:106-154). */
int sb_rope_correct_scatter_paged_layers(const uint64_t* kv_layer_ptrs,
                                         const uint64_t* donor_layer_ptrs, int64_t num_layers,
                                         const int32_t* block_table, const int32_t* donor_pos,
                                         const int32_t* target_pos, const float* inv_freq,
                                         int64_t num_pairs, int64_t num_heads,
                                         int64_t block_size, int64_t head_dim,
                                         int64_t donor_seq_len, int64_t num_blocks_total,
                                         int64_t num_blocks_per_seq, const int64_t* kv_strides,
                                         const int64_t* d_strides, int32_t dtype,
                                         int32_t flags, void* stream);

/* Composite (multi-donor) scatter over many layers in one pass: pair i moves the rows of
 * donor donor_index[i] at position donor_pos[i] (K and V, every layer and head) to
 * target_pos[i] of the paged caches, rotating K by (target_pos - donor_pos) when inv_freq
 * is not NULL (plain copy when it is).
 *   donor_layer_ptrs  device [num_donors * num_layers] base addresses (donor-major), each a
 *                     [2, H, S_k, D] tensor, 16-byte aligned
 *   donor_strides     host [num_donors * 5]: kv, head and sequence strides of donor k in
 *                     elements, the rows S_k its tensor holds, and the sequence position of
 *                     its row 0 (0 for a whole donor; c * T for a staged chunk c): the pair
 *                     reads row donor_pos[i] - first, and K is still rotated by
 *                     target_pos[i] - donor_pos[i]
 * Pairs whose donor index, donor position or target slot is out of range are skipped.
 * Target positions must be distinct across all pairs (a composite plan gives each target
 * position one donor); duplicates race. Donors are moved in launches of at most 16.
 * flags: as for sb_scatter_donor_kv_paged_layers.
 * No reference counterpart: the reference carries the per-position donor map
 * (semblend_core/partial_attention.py:306-435, multi_donor_types.py:50-78) but loads and
 * scatters one donor at a time (synapse_kv_connector/semblend_connector.py:1508-1701). */
int sb_composite_scatter_paged_layers(const uint64_t* kv_layer_ptrs, int64_t num_layers,
                                      const uint64_t* donor_layer_ptrs, int64_t num_donors,
                                      const int64_t* donor_strides, const int32_t* donor_index,
                                      const int32_t* donor_pos, const int32_t* target_pos,
                                      const float* inv_freq, int64_t num_pairs,
                                      int64_t num_heads, int64_t block_size, int64_t head_dim,
                                      const int32_t* block_table, int64_t num_blocks_total,
                                      int64_t num_blocks_per_seq, const int64_t* kv_strides,
                                      int32_t dtype, int32_t flags, void* stream);

/* sb_composite_scatter_paged_layers with the pairs grouped by donor instead of a per-pair
 * donor index: donor k's pairs occupy [segment_ends[k-1], segment_ends[k]) of donor_pos /
 * target_pos (segment_ends: host [num_donors], each end but the last a multiple of 256, the
 * last equal to num_pairs; a segment is padded with pairs whose positions are -1, which are
 * skipped). Every workgroup's pairs then share one donor, so its strides and layer table are
 * read once per workgroup instead of once per pair. At most 16 donors. Same results as the
 * indexed form. No reference counterpart (see sb_composite_scatter_paged_layers). */
int sb_composite_scatter_paged_layers_grouped(const uint64_t* kv_layer_ptrs,
                                              int64_t num_layers,
                                              const uint64_t* donor_layer_ptrs,
                                              int64_t num_donors,
                                              const int64_t* donor_strides,
                                              const int64_t* segment_ends,
                                              const int32_t* donor_pos,
                                              const int32_t* target_pos,
                                              const float* inv_freq, int64_t num_pairs,
                                              int64_t num_heads, int64_t block_size,
                                              int64_t head_dim, const int32_t* block_table,
                                              int64_t num_blocks_total,
                                              int64_t num_blocks_per_seq,
                                              const int64_t* kv_strides, int32_t dtype,
                                              int32_t flags, void* stream);

/* Flat RoPE correction over k [L, H, S, D] (k_strides[4]; pass L = 1 for [H, S, D]):
 * for each pair i in order, the row at donor position d_i is rotated by (t_i - d_i) and
 * rounded to dtype; rows hit by several pairs are rotated once per pair, in pair order.
 * out may equal k (in place); when out != k, rows no pair touches are copied unchanged.
 * workspace: device int32 array of 2 * S entries (scratch for the per-row pair index).
 * Replaces semblend_core/rope_correction.py:336-399 (rope_correct_k). */
int sb_rope_correct_k(void* out, const void* k, const int32_t* donor_pos,
                      const int32_t* target_pos, const float* inv_freq, int32_t* workspace,
                      int64_t num_pairs, int64_t num_layers, int64_t num_heads, int64_t seq_len,
                      int64_t head_dim, const int64_t* out_strides, const int64_t* k_strides,
                      int32_t dtype, void* stream);

/* In-place sb_rope_correct_k for callers that guarantee that no donor position repeats
 * (for instance the identity d = 0..S-1 of a whole-sequence correction): one thread group per
 * pair rotates the rows at its donor position, with no per-position index and no workspace,
 * so a call is one launch. Repeated donor positions race here; use sb_rope_correct_k for
 * them. Same rotation and rounding as sb_rope_correct_k.
 * Replaces semblend_core/rope_correction.py:336-399 for distinct donor positions. */
int sb_rope_correct_k_distinct(void* k, const int32_t* donor_pos, const int32_t* target_pos,
                               const float* inv_freq, int64_t num_pairs, int64_t num_layers,
                               int64_t num_heads, int64_t seq_len, int64_t head_dim,
                               const int64_t* k_strides, int32_t dtype, void* stream);

/* In-place rotation of K rows in a paged cache by one delta:
 *   K[bt[p / bs], h, p % bs, :] = R(delta) K[...], applied repeat[i] times (rounded to dtype
 *   after each application) for positions[i]. repeat may be NULL (once each).
 * k_plane points at the K plane; k_strides[4] = (block, head, pos, dim), so both the
 * [NB, 2, H, bs, D] and the vLLM [2, NB, bs, H, D] layouts are addressed.
 * Replaces semblend_core/rope_correction.py:699-783 (apply_rope_delta_inplace). */
int sb_apply_rope_delta_inplace(void* k_plane, const int32_t* block_table,
                                const int32_t* positions, const int32_t* repeat,
                                int64_t num_positions, int64_t delta, const float* inv_freq,
                                int64_t num_heads, int64_t block_size, int64_t head_dim,
                                int64_t num_blocks_total, int64_t num_blocks_per_seq,
                                const int64_t* k_strides, int32_t dtype, void* stream);

/* sb_apply_rope_delta_inplace with positions (and repeat, or NULL) in HOST memory, at most
 * SB_INLINE_POSITIONS_MAX of them: they are copied into the launch's own argument block, so
 * a short list needs no device buffer and no host-to-device copy (the per-call cost of the
 * reference's caller pattern, one call per distinct delta). Same results as
 * sb_apply_rope_delta_inplace; more positions are rejected with SB_ERR_INVALID_ARGUMENT.
 * The host arrays may be reused as soon as the call returns.
 * Replaces semblend_core/rope_correction.py:699-783 (apply_rope_delta_inplace) for short
 * position lists. */
int sb_apply_rope_delta_inplace_host(void* k_plane, const int32_t* block_table,
                                     const int32_t* positions, const int32_t* repeat,
                                     int64_t num_positions, int64_t delta,
                                     const float* inv_freq, int64_t num_heads,
                                     int64_t block_size, int64_t head_dim,
                                     int64_t num_blocks_total, int64_t num_blocks_per_seq,
                                     const int64_t* k_strides, int32_t dtype, void* stream);

/* In-place rotation of the K rows of many layers' paged caches, one delta per position, in
 * one launch: for every layer l and i < num_positions,
 *   K_l[bt[p / bs], h, p % bs, :] = R(deltas[i]) K_l[...],  p = positions[i].
 * kv_layer_ptrs: device array of num_layers K-plane base addresses (16-byte aligned), all
 * caches sharing k_strides[4] = (block, head, pos, dim) and dtype. Positions must be distinct
 * within one call (rows are rotated concurrently); positions past the block table or in an
 * invalid physical block are skipped. |deltas[i]| < 2^31.
 * Replaces the per-(layer, pair) loop of apply_rope_delta_inplace calls in
 * semblend/integration/trtllm/semblend_provider.py:305-318 and the one-call-per-delta loop
 * over semblend_core/rope_correction.py:699-783 (apply_rope_delta_inplace). */
int sb_apply_rope_deltas_inplace_layers(const uint64_t* kv_layer_ptrs, int64_t num_layers,
                                        const int32_t* block_table, const int32_t* positions,
                                        const int32_t* deltas, int64_t num_positions,
                                        const float* inv_freq, int64_t num_heads,
                                        int64_t block_size, int64_t head_dim,
                                        int64_t num_blocks_total, int64_t num_blocks_per_seq,
                                        const int64_t* k_strides, int32_t dtype, void* stream);

/* sb_apply_rope_deltas_inplace_layers with positions and deltas in HOST memory, at most
 * SB_INLINE_POSITIONS_MAX of them: they travel in the launch's own argument block (no device
 * buffer, no host-to-device copy; a launch recorded into a HIP graph holds them). Same results;
 * more positions are rejected with SB_ERR_INVALID_ARGUMENT. The host arrays may be reused as
 * soon as the call returns. Replaces the same reference loops as the device form. */
int sb_apply_rope_deltas_inplace_layers_host(const uint64_t* kv_layer_ptrs, int64_t num_layers,
                                             const int32_t* block_table,
                                             const int32_t* positions, const int32_t* deltas,
                                             int64_t num_positions, const float* inv_freq,
                                             int64_t num_heads, int64_t block_size,
                                             int64_t head_dim, int64_t num_blocks_total,
                                             int64_t num_blocks_per_seq,
                                             const int64_t* k_strides, int32_t dtype,
                                             void* stream);

/* Permutation inside a paged cache with snapshot semantics: every source row (K and V) is
 * read before any target row is written; V is copied, K rotated by (tgt - src).
 * workspace: device buffer of num_pairs * 2 * H * D elements of dtype.
 * Replaces semblend_core/rope_correction.py:407-476 (permute_paged_kv_with_rope). */
int sb_permute_paged_kv_with_rope(void* kv_cache, const int32_t* block_table,
                                  const int32_t* src_pos, const int32_t* tgt_pos,
                                  const float* inv_freq, void* workspace, int64_t num_pairs,
                                  int64_t num_heads, int64_t block_size, int64_t head_dim,
                                  int64_t num_blocks_total, int64_t num_blocks_per_seq,
                                  const int64_t* kv_strides, int32_t dtype, void* stream);

/* NoPE two-step permutation: K at each target = R(tgt) R(-src) K_snapshot(src) (two fp32
 * rotations, one rounding); V rows copied from v_src_pos to v_tgt_pos after a snapshot.
 * The host resolves the reference's sequential V copies into (v_src, v_tgt) pairs.
 * workspace: device buffer of (num_pairs + num_v_pairs) * H * D elements of dtype.
 * Replaces semblend_core/rope_correction.py:599-697 (kernel :496-596, CPU path :786-823). */
int sb_nope_permute_paged_kv(void* kv_cache, const int32_t* block_table,
                             const int32_t* src_pos, const int32_t* tgt_pos, int64_t num_pairs,
                             const int32_t* v_src_pos, const int32_t* v_tgt_pos,
                             int64_t num_v_pairs, const float* inv_freq, void* workspace,
                             int64_t num_heads, int64_t block_size, int64_t head_dim,
                             int64_t num_blocks_total, int64_t num_blocks_per_seq,
                             const int64_t* kv_strides, int32_t dtype, void* stream);

/* Multi-layer forms of the two permutations above, for the production vLLM path, which
 * corrects every layer of a request with the same permutation: one launch pair (snapshot,
 * write) covers all layers. kv_layer_ptrs: device array of num_layers per-layer cache base
 * addresses (16-byte aligned), all with the element strides kv_strides[5] in
 * (block, kv, head, pos, dim) order, so the vLLM flash-attn [2, NB, bs, H, D], TRT-LLM
 * [NB, 2, tpb, H, D] and standard [NB, 2, H, bs, D] caches are all addressed without a copy.
 * workspace: num_layers times the single-layer size (layer-major snapshot).
 * Replace the per-layer loop of synapse_kv_connector/model_runner_hook.py:519-585 around
 * rope_correction.py:407-476 (delta) and :599-697 (NoPE); the reference decodes every cache
 * as [NB, 2, H, bs, D] (rope_correction.py:432, :623), which the strides here make exact. */
int sb_permute_paged_kv_with_rope_layers(const uint64_t* kv_layer_ptrs, int64_t num_layers,
                                         const int32_t* block_table, const int32_t* src_pos,
                                         const int32_t* tgt_pos, const float* inv_freq,
                                         void* workspace, int64_t num_pairs, int64_t num_heads,
                                         int64_t block_size, int64_t head_dim,
                                         int64_t num_blocks_total, int64_t num_blocks_per_seq,
                                         const int64_t* kv_strides, int32_t dtype,
                                         void* stream);
int sb_nope_permute_paged_kv_layers(const uint64_t* kv_layer_ptrs, int64_t num_layers,
                                    const int32_t* block_table, const int32_t* src_pos,
                                    const int32_t* tgt_pos, int64_t num_pairs,
                                    const int32_t* v_src_pos, const int32_t* v_tgt_pos,
                                    int64_t num_v_pairs, const float* inv_freq, void* workspace,
                                    int64_t num_heads, int64_t block_size, int64_t head_dim,
                                    int64_t num_blocks_total, int64_t num_blocks_per_seq,
                                    const int64_t* kv_strides, int32_t dtype, void* stream);

/* ------------------------------------------------------------------------------------------
 * Partial-prefill attention (causal; row at position p attends to keys 0..p)
 * ---------------------------------------------------------------------------------------- */

/* Dense drop-in: out[h, i, :] = softmax(scale * q[h, i] . k[h, :i+1]) v[h, :i+1] for every i
 * with compute_mask[i] != 0, and 0 elsewhere. q, k, v, out are [H, S, D] with strides
 * (head, seq, dim) given in q_strides[3], k_strides[3], v_strides[3] and o_strides[3].
 * compute_mask: device uint8 array of S entries. The rows are compacted on the device, so the
 * call never synchronises with the host. Rows whose mask is 0 are written as zeros.
 * workspace: device buffer of sb_partial_prefill_attention_workspace_size(...) bytes.
 * Replaces semblend_core/triton_kernels.py:655-734 (kernel :531-652, CPU path :717-732). */
int64_t sb_partial_prefill_attention_workspace_size(int64_t num_heads, int64_t seq_len,
                                                    int64_t head_dim, int32_t dtype);
int sb_partial_prefill_attention(void* out, const void* q, const void* k, const void* v,
                                 const uint8_t* compute_mask, void* workspace,
                                 int64_t workspace_bytes, int64_t num_heads, int64_t seq_len,
                                 int64_t head_dim, float scale, const int64_t* q_strides,
                                 const int64_t* k_strides, const int64_t* v_strides,
                                 const int64_t* o_strides, int32_t dtype, void* stream);

/* GQA attention over a paged cache for a compact set of query rows:
 *   out[r, hq, :] = softmax(scale * q[r, hq] . K[hkv, 0..p_r]) V[hkv, 0..p_r],
 *   hkv = hq / (num_q_heads / num_kv_heads), p_r = positions[r].
 * q and out are [R, Hq, D] (q_strides[3], o_strides[3] = (row, head, dim));
 * kv_cache [NB, 2, Hkv, bs, D] with kv_strides[5] = (block, kv, head, pos, dim).
 * positions should be ascending (any order is correct; ascending is fastest).
 * workspace: device buffer of sb_partial_attention_paged_workspace_size(...) bytes (fp32
 * partials of the split key range; the size may be 0, then workspace may be NULL).
 * No reference counterpart: the reference attention is MHA over contiguous K/V
 * (semblend_core/triton_kernels.py:655-734); this is the GQA + paged form its callers need. */
int64_t sb_partial_attention_paged_workspace_size(int64_t num_rows, int64_t num_q_heads,
                                                  int64_t num_kv_heads, int64_t head_dim,
                                                  int64_t block_size,
                                                  int64_t num_blocks_per_seq, int32_t dtype);
int sb_partial_attention_paged(void* out, const void* q, const void* kv_cache,
                               const int32_t* block_table, const int32_t* positions,
                               void* workspace, int64_t workspace_bytes, int64_t num_rows,
                               int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                               int64_t block_size, int64_t num_blocks_total,
                               int64_t num_blocks_per_seq, float scale,
                               const int64_t* q_strides, const int64_t* o_strides,
                               const int64_t* kv_strides, int32_t dtype, void* stream);

/* Host-planned form of sb_partial_attention_paged. A caller that knows the query positions on
 * the host (they come from the reuse plan, and one request's positions serve every layer)
 * plans once: sb_partial_attention_paged_plan reads the HOST positions and writes into `plan`
 * (capacity int32 entries) the key split {ks_first, ks_rest, max_chunks} followed by the
 * dispatch order of every work item, longest first (a row tile's first key chunk of ks_first
 * keys, its later chunks of ks_rest keys, chosen by a longest-first schedule model of the
 * launch). With plan == NULL it returns the number of entries needed; otherwise the number
 * written, or a negative SB_ERR_INVALID_ARGUMENT on bad arguments. For a dtype / head_dim
 * the MFMA kernel does not take, max_chunks is 0 and there are no items.
 * sb_partial_attention_paged_planned takes the device copy of the item order (plan + 3), its
 * length (refused unless it is max_chunks * ceil(num_rows * group / 128) * num_kv_heads,
 * the launch's item count) and the three split values, otherwise the arguments of
 * sb_partial_attention_paged; its
 * workspace is sb_partial_attention_paged_planned_workspace_size(...) bytes. The order only
 * schedules the launch: it names every item whatever the positions hold, so results are
 * correct for any positions (the same within the attention bar as the unplanned entry; the
 * split-key partials round differently), and fastest for the positions it was planned from.
 * No reference counterpart (see sb_partial_attention_paged). */
int64_t sb_partial_attention_paged_plan(const int32_t* positions, int64_t num_rows,
                                        int64_t num_q_heads, int64_t num_kv_heads,
                                        int64_t head_dim, int64_t block_size,
                                        int64_t num_blocks_per_seq, int32_t dtype,
                                        int32_t* plan, int64_t capacity);
int64_t sb_partial_attention_paged_planned_workspace_size(int64_t num_rows,
                                                          int64_t num_q_heads,
                                                          int64_t num_kv_heads,
                                                          int64_t head_dim, int32_t max_chunks,
                                                          int32_t dtype);
int sb_partial_attention_paged_planned(void* out, const void* q, const void* kv_cache,
                                       const int32_t* block_table, const int32_t* positions,
                                       const int32_t* item_order, int64_t num_items,
                                       int32_t ks_first, int32_t ks_rest,
                                       int32_t max_chunks, void* workspace,
                                       int64_t workspace_bytes, int64_t num_rows,
                                       int64_t num_q_heads, int64_t num_kv_heads,
                                       int64_t head_dim, int64_t block_size,
                                       int64_t num_blocks_total, int64_t num_blocks_per_seq,
                                       float scale, const int64_t* q_strides,
                                       const int64_t* o_strides, const int64_t* kv_strides,
                                       int32_t dtype, void* stream);

/* No-allocation form of sb_partial_attention_paged, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments minus the workspace, same kernels, same plan and bit-identical
 * results; the split-key partials live in a fixed array inside the library, one per GPU,
 * of sb_partial_attention_paged_noalloc_max_scratch() bytes (128 MiB), held from module load
 * until the process ends. A call whose partials would exceed it fails with
 * SB_ERR_INVALID_ARGUMENT before any launch. Calls on one GPU share that GPU's array:
 * calls that overlap on one GPU (concurrent streams, or threads) race and must be
 * serialised by the caller. Nothing in the array needs clearing between calls. The call
 * makes no hipMalloc/hipFree or allocating library call.
 * No reference counterpart (the reference has no paged GQA attention entry). */
int64_t sb_partial_attention_paged_noalloc_max_scratch(void);
int sb_partial_attention_paged_noalloc(void* out, const void* q, const void* kv_cache,
                                       const int32_t* block_table, const int32_t* positions,
                                       int64_t num_rows, int64_t num_q_heads,
                                       int64_t num_kv_heads, int64_t head_dim,
                                       int64_t block_size, int64_t num_blocks_total,
                                       int64_t num_blocks_per_seq, float scale,
                                       const int64_t* q_strides, const int64_t* o_strides,
                                       const int64_t* kv_strides, int32_t dtype, void* stream);

/* Batched GQA attention over a paged cache: num_reqs requests share kv_cache, request r
 * has rows_per_req[r] query rows and the first blocks_per_req[r] entries of block-table row
 * block_tables[r * block_table_stride ...]. q, out and positions hold the requests' rows back
 * to back (positions are within each request). rows_per_req and blocks_per_req are HOST
 * arrays: the launch plan is built on the host, so the call never synchronises. Requests run
 * longest context first, up to 16 per launch; the result equals one
 * sb_partial_attention_paged call per request.
 * workspace: device buffer of sb_partial_attention_paged_varlen_workspace_size(...) bytes
 * (may be 0, then workspace may be NULL).
 * No reference counterpart: the reference runs one request per call; this replaces the
 * per-request loop of its callers (synapse_kv_connector/model_runner_hook.py:519-585 walks
 * one request's layers per hook). */
int64_t sb_partial_attention_paged_varlen_workspace_size(int64_t num_reqs,
                                                         const int64_t* rows_per_req,
                                                         const int64_t* blocks_per_req,
                                                         int64_t num_q_heads,
                                                         int64_t num_kv_heads,
                                                         int64_t head_dim, int64_t block_size,
                                                         int32_t dtype);
int sb_partial_attention_paged_varlen(void* out, const void* q, const void* kv_cache,
                                      const int32_t* block_tables, int64_t block_table_stride,
                                      const int32_t* positions, int64_t num_reqs,
                                      const int64_t* rows_per_req,
                                      const int64_t* blocks_per_req, void* workspace,
                                      int64_t workspace_bytes, int64_t num_q_heads,
                                      int64_t num_kv_heads, int64_t head_dim,
                                      int64_t block_size, int64_t num_blocks_total, float scale,
                                      const int64_t* q_strides, const int64_t* o_strides,
                                      const int64_t* kv_strides, int32_t dtype, void* stream);

/* ------------------------------------------------------------------------------------------
 * Flat device copy (measurement reference; no reference counterpart)
 * ---------------------------------------------------------------------------------------- */

/* dst[0:num_bytes) = src[0:num_bytes): one 16-byte vector per thread with nontemporal loads
 * and stores, the achievable HBM rate the row movers are compared with. Both buffers must be
 * 16-byte aligned and num_bytes a multiple of 16; the buffers must not overlap. Logged by the
 * kernel timing below under "copy". */
int sb_device_copy(void* dst, const void* src, int64_t num_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * Kernel timing (instrumentation for benchmarks; no reference counterpart)
 * ---------------------------------------------------------------------------------------- */

/* enable != 0 clears the timing log and starts attaching a pair of HIP timing events to every
 * launch of the library's kernels (hipExtLaunchKernel start/stop events, stamped with the
 * kernel's own start and end, so no extra work enters the stream); enable == 0 stops logging
 * (the log stays readable). At most 65536 launches are logged. Kernel names:
 * "move_rows", "rope_rows", "rope_index", "fill_i32", "attn_mfma", "attn_valu", "attn_merge",
 * "mask_compact", "zero_rows", "copy". */
int sb_kernel_timing_enable(int32_t enable);

/* Sum of the logged durations (ms) and number of logged launches of one kernel. Waits for the
 * logged events to complete. */
int sb_kernel_timing_read(const char* kernel, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* SEMBLEND_HIP_H */
