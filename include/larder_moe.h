/* larder_moe.h: C ABI of the MI355X (gfx950) routed-expert MoE layer over GGUF Q4_0 / Q4_K blocks.
 *
 * Every entry point:
 *   - takes device pointers and plain sizes, and a hipStream_t passed as void* (NULL = the null stream);
 *   - only enqueues work on that stream: no host synchronisation, no allocation;
 *   - returns 0 on success, a positive hipError_t when a HIP call failed, or a negative LMOE_E* code when an
 *     argument was refused; lmoe_error() then returns a one-sentence reason (thread-local).
 * Expert buffers are the reference's arena layout: uint8 [n_experts][rows][row bytes] with row bytes
 * cols / 32 * 18 (Q4_0) or cols / 256 * 144 (Q4_K), 16-byte aligned (stream_fast.py:3936-3941).
 * Workspaces are caller-owned device memory sized by the matching *_workspace_bytes query; their contents on entry
 * do not matter.
 */
#ifndef LARDER_MOE_H
#define LARDER_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of activations, logits and outputs */
enum { LMOE_F32 = 0, LMOE_F16 = 1, LMOE_BF16 = 2 };
/* ggml block types, by ggml type id (gguf_ref.py:8-15) */
enum { LMOE_Q4_0 = 2, LMOE_Q4_1 = 3, LMOE_Q8_0 = 8, LMOE_Q4_K = 12, LMOE_Q5_K = 13, LMOE_Q6_K = 14 };
/* Q4_0 and Q4_K run on every kernel. Q4_1, Q8_0, Q5_K and Q6_K run on the general decode chain
 * (lmoe_gemv_gate_up / lmoe_gemv_down_combine with raw x and float32 h: one lane a 32-weight chunk,
 * gguf_experts.py:78-373's task decoders restated), in lmoe_dequant, and on the grouped path through
 * lmoe_dequant_gemm_f16 + lmoe_grouped_*_f16w; the prepared-row entry points take Q4_0 and Q4_K only. */
/* refusals */
enum { LMOE_EINVAL = -1, LMOE_ETYPE = -2, LMOE_ESHAPE = -3, LMOE_EALIGN = -4, LMOE_EWORKSPACE = -5 };

/* The reason for the last nonzero return on this thread ("" if none). */
const char *lmoe_error(void);
/* ABI version, bumped on any signature change. */
int lmoe_abi_version(void);

/* Kernel-exact timing for benchmarks (no counterpart in the reference): after lmoe_profile_arm(n), the next n
 * kernels this thread launches through the library (router, top-k, gate/up, down, grouping, grouped GEMMs,
 * combine) are each bracketed by a start / stop event pair recorded at the kernel's own begin and end
 * (hipExtLaunchKernelGGL); lmoe_profile_read waits for them, writes each launch's duration in launch order into
 * ms[0 .. min(count, cap)), the number recorded into *count, and disarms. Not for use under graph capture. */
int lmoe_profile_arm(int max_launches);
int lmoe_profile_read(float *ms, int cap, int *count);

/* Per-workgroup phase timeline of the decode kernels, for benchmarks (no counterpart in the reference). After
 * lmoe_timeline_arm(buf, rows) (buf: device memory, rows x 8 uint64, zeroed by the caller), the router GEMV
 * (lmoe_router_gemv), the fused gate/up (lmoe_moe_gate_up*) and the two-wavefront down (lmoe_gemv_down_combine_prepped)
 * that this thread launches, also into a graph under capture, run their stamping forms (the same results bit for
 * bit): each workgroup writes the device wall clock (lmoe_timeline_clock_khz ticks a millisecond) into its row at
 * each phase it reaches: 0 start, 1 inputs in (gate/up: its logits row; down: the token's ids), 2 top-k done
 * (gate/up), 3 weights in, 4 end; a phase not reached stays as the caller left it. Each launch takes the next rows in
 * launch order (grid x fastest, then y); a launch that does not fit runs unstamped and is not listed.
 * lmoe_timeline_disarm writes the number of listed launches into *count and stops stamping new launches (a captured
 * graph keeps stamping on every replay); lmoe_timeline_launch(i) gives listed launch i's kernel (1 router, 2 gate/up,
 * 3 down), its first row and its workgroup count. */
int lmoe_timeline_arm(unsigned long long *buf, long long rows);
int lmoe_timeline_disarm(int *count);
int lmoe_timeline_launch(int i, int *kernel, long long *row0, int *n_wg);
int lmoe_timeline_clock_khz(int *khz);

/* Router top-k over given logits. Replaces route_cuda.probs (route_cuda.py:280-288; kernel moe_probs
 * route_cuda.py:193-254) and the block's softmax/argpartition/take/renorm ops (stream_fast.py:4352-4370).
 * logits [T][E] in ldtype -> ids [T][k] best first (ties: lowest expert index), scores [T][k] fp32 softmax
 * probabilities of the picked experts, renormalised to sum 1 when norm != 0. E <= 1024, k <= 32. */
int lmoe_router_topk(const void *logits, int ldtype, int T, int E, int k, int norm, uint32_t *ids, float *scores,
                     void *stream);

/* lmoe_router_topk and lmoe_to_gemm_f16 in ONE launch (no counterpart in the reference; the prefill chain's two steps
 * before the grouping when the logits are given, stream_fast.py:4352-4370 / gguf_experts.py:698-722): ids / scores
 * [T][k] from logits [T][E] as lmoe_router_topk gives them, and x [n] (n % 32 == 0, 16-byte aligned) to xh [n] in f16
 * in the grouped GEMMs' K order as lmoe_to_gemm_f16 gives it, bit for bit. One kernel boundary fewer. */
int lmoe_topk_and_gemm_f16(const void *logits, int ldtype, int T, int E, int k, int norm, uint32_t *ids,
                           float *scores, const void *x, int xdtype, long long n, void *xh, void *stream);

/* lmoe_router_topk on fp32 logits [T][E] with a folded shared expert's m slices appended to every token (no
 * counterpart in the reference; the prefill form of lmoe_moe_gate_up_ext's slots): ids / scores [T][k + m], slot
 * k + j = (E + j, sigmoid(gate[t])), gate [T] the shared expert's gate logits (lmoe_router_gemm's gate output). The
 * grouped GEMMs then run the slices as experts E .. E + m - 1 of the extended weight buffers. k + m <= 64. */
int lmoe_router_topk_shared(const float *logits, int T, int E, int k, int norm, const float *gate, int m,
                            uint32_t *ids, float *scores, void *stream);

/* Prepared activation rows: an activation row of 64 P values as P units of 36 dwords (32 dwords of f16 pairs in
 * the nibble order of block type qtype, the sums of the unit's two 32-value halves as fp32, two zero dwords), the
 * form the expert kernels read. x [rows][H] in xdtype -> xprep [rows][H / 64 * 36] uint32.
 * Range: every value is rounded to f16 once (exact for f16 x, and for bf16 x inside f16's normal range), so an |x|
 * above 65504 becomes inf, and so does an |h| above 65504 in the prepared h rows the gate/up entries write: the
 * expert rows fed by such a value come out non-finite. The reference stages x and h as f32 (gguf_experts.py:452-526);
 * the general kernels (raw x, fp32 h) keep that range. */
int lmoe_prep_x(const void *x, int xdtype, int rows, int H, int qtype, uint32_t *xprep, void *stream);

/* Router GEMV: logits[t][e] = x[t] . wr[e] (fp32 accumulation), and when wsg is given the shared-expert gate logit
 * x[t] . wsg as logits[t][E] (row stride E + 1 then); when xprep is given, also x's prepared rows for block type
 * qtype. Replaces the block's gate linear (stream_fast.py:4358) and shared_expert_gate (:4375).
 * x [T][H] in xdtype, wr [E][H] and wsg [H] in wdtype (F16, BF16 or F32), T <= 16, H % 64 == 0. */
int lmoe_router_gemv(const void *x, int xdtype, const void *wr, const void *wsg, int wdtype, int T, int H, int E,
                     float *logits, uint32_t *xprep, int qtype, void *stream);

/* lmoe_router_gemv then lmoe_router_topk on its logits: the decode rows of route_cuda.probs after the gate linear
 * (route_cuda.py:433-444). */
int lmoe_router_gemv_topk(const void *x, int xdtype, const void *wr, const void *wsg, int wdtype, int T, int H,
                          int E, int k, int norm, float *logits, uint32_t *ids, float *scores, uint32_t *xprep,
                          int qtype, void *stream);

/* Router GEMV and top-k in ONE launch: the logits of lmoe_router_gemv (the same bits: every row summed in its order),
 * then the ids / scores of lmoe_router_topk (ties to the lowest index, best first), plus the prepared activation rows
 * when xprep is given. The workgroup that finishes its rows last ranks every token, so no gate/up wavefront has to
 * rank (the fused form lmoe_moe_gate_up ranks in each of them). ks: slots a token in ids / scores, k or (with wsg)
 * k + m, slots k + j then holding id E + j and weight sigmoid(x . wsg): the folded shared expert's slices of
 * lmoe_moe_gate_up_ext.
 * sync: one uint32 of device memory, zero before the first call, left zero by each call; one per stream (two calls
 * in flight on one counter race). E <= 512, k <= 16, T <= 16. Replaces the reference's gate linear + moe_probs
 * (route_cuda.py:193-254, 280-288, 433-444). */
int lmoe_router_gemv_rank(const void *x, int xdtype, const void *wr, const void *wsg, int wdtype, int T, int H, int E,
                          int k, int norm, int ks, float *logits, uint32_t *ids, float *scores, uint32_t *xprep,
                          int qtype, uint32_t *sync, void *stream);

/* The cache-biased route of route_cuda.route / route_cuda.bias_probs (route_cuda.py:42-121, 158-178, 306-417), which
 * reproduce CacheBiasedMoE._select: per row of gates g [E] in gdtype T (softmax: the row holds logits and
 * g = T(softmax)), spread = T(max g - min g), rank = float(g) + float(T(T(lam) * spread)) * m with m = mask[e]
 * (mask NULL: table mode, m = 0 <= slot_of[e] < lim), inds = the k largest of rank with MLX's rule (equal values to
 * the LARGER index; the k ascending, best last). With tau > 0 the budget: honest = the same on g, the two k-gate
 * sums in T in MLX's row_reduce order, and honest replaces inds when T(m_h - m_b) > T(T(tau) * m_h).
 * Outputs: inds [T][k] uint32; with slot_of: rhs [T][k] = max(slot_of[inds], 0) and ok [1] = all(slot_of[inds] >= 0)
 * (either may be NULL); scores [T][k] in gdtype = the picked gates, divided by their sum (taken in output order in
 * T) when norm, or NULL. T <= 16, E <= 1024, k <= 32. */
int lmoe_route_bias(const void *gates, int gdtype, int T, int E, int k, const float *mask, const int32_t *slot_of,
                    int lim, float lam, float tau, int softmax, int norm, uint32_t *inds, uint32_t *ok, int32_t *rhs,
                    void *scores, void *stream);

/* Decode chain, gate/up: h[s][i] = silu(x[s / topk] . wg[slots[s]][i]) * (x[s / topk] . wu[slots[s]][i]),
 * fp32. Replaces gguf_experts kernel gguf_gate_up (gguf_experts.py:452-495) as driven by _chain
 * (gguf_experts.py:610-623). x [n_slots / topk][H] in xdtype; slots >= n_experts give h rows of zeros.
 * H % 64 == 0 (Q4_0) or H % 256 == 0 (Q4_K). */
int lmoe_gemv_gate_up(const void *x, int xdtype, const uint32_t *slots, int n_slots, int topk, const uint8_t *wg,
                      const uint8_t *wu, int type_g, int type_u, int n_experts, int H, int I, float *h,
                      void *stream);

/* lmoe_gemv_gate_up on prepared rows: xg_prep (and xu_prep when type_u differs from type_g) [n_slots / topk][...];
 * writes h (fp32, may be NULL) and / or hprep, h's prepared rows for the down matrix's type_d without their sums
 * ([n_slots][I / 64 * 36], may be NULL; type_d Q4_0, Q4_K, Q6_K (which takes the Q4_K order) or Q8_0 (the Q4_0
 * order)). */
int lmoe_gemv_gate_up_prepped(const uint32_t *xg_prep, const uint32_t *xu_prep, const uint32_t *slots, int n_slots,
                              int topk, const uint8_t *wg, const uint8_t *wu, int type_g, int type_u, int n_experts,
                              int H, int I, float *h, uint32_t *hprep, int type_d, void *stream);

/* The decode layer's gate/up with the router's top-k fused in: each workgroup ranks its token's logits
 * [T][ld_stride] (as lmoe_router_topk: ties to the lowest expert index, softmax scores, renormalised when norm),
 * takes its slot's expert, writes ids [T][k] and scores [T][k], and runs lmoe_gemv_gate_up_prepped's work on
 * prepared rows xg_prep / xu_prep [T][...] into hprep [T * k][I / 64 * 36]. Replaces route_cuda.probs plus
 * gguf_gate_up on decode rows (route_cuda.py:433-444; gguf_experts.py:452-495). E <= 1024, k <= 32. */
int lmoe_moe_gate_up(const float *logits, int ld_stride, int T, int k, int norm, const uint32_t *xg_prep,
                     const uint32_t *xu_prep, const uint8_t *wg, const uint8_t *wu, int type_g, int type_u,
                     int n_experts, int H, int I, uint32_t *ids, float *scores, uint32_t *hprep, int type_d,
                     void *stream);

/* lmoe_moe_gate_up with the layer's shared expert folded in as m = with_shared more slots a token (0 is
 * lmoe_moe_gate_up): a shared expert m times the routed width, cut into m slices of its intermediate features
 * (slice j: gate / up rows [j I, (j + 1) I), down columns likewise), stored as experts n_experts .. n_experts + m - 1
 * of wg / wu (same shape and type as the routed ones); logits rows hold the shared expert's gate logit at column
 * n_experts (the router GEMV's row E), and each token gets k + m slots: ids / scores [T][k + m] with slot k + j =
 * (n_experts + j, sigmoid(gate logit)), hprep [T (k + m)][I / 64 * 36]. lmoe_gemv_down_combine_prepped with k + m
 * and wd of n_experts + m experts then weights the slices like routed experts, and their sum is the gated shared
 * row: three launches a layer instead of five. Takes the register-resident form (H = 2048 or 4096, one type for
 * gate and up), k + m <= 64. No counterpart in the reference (its shared expert is MLX ops,
 * stream_fast.py:4403-4405). */
int lmoe_moe_gate_up_ext(const float *logits, int ld_stride, int T, int k, int norm, const uint32_t *xg_prep,
                         const uint32_t *xu_prep, const uint8_t *wg, const uint8_t *wu, int type_g, int type_u,
                         int n_experts, int H, int I, uint32_t *ids, float *scores, uint32_t *hprep, int type_d,
                         int with_shared, void *stream);

/* lmoe_moe_gate_up (with_shared = 0) or lmoe_moe_gate_up_ext (with_shared = m slices) writing h as fp32
 * [T (k + m)][I] instead of prepared rows, for a layer whose down matrix is a type beyond Q4_0 / Q4_K (the 35B's
 * Q6_K down): lmoe_gemv_down_combine then takes h. One Q4 type for gate and up, hidden 2048 or 4096, I even (the
 * register-resident form). Replaces route_cuda.probs plus gguf_gate_up on decode rows with f32 h out, as the
 * reference's chain passes it (route_cuda.py:433-444; gguf_experts.py:452-495, 600-653). */
int lmoe_moe_gate_up_h(const float *logits, int ld_stride, int T, int k, int norm, const uint32_t *x_prep,
                       const uint8_t *wg, const uint8_t *wu, int type, int n_experts, int H, int I, uint32_t *ids,
                       float *scores, float *h, int with_shared, void *stream);

/* Decode chain, down with the weighted combine fused:
 *   out[t][n] = sum_j scores[t][j] * (h[t * k + j] . wd[ids[t][j]][n])
 *               (+ sigmoid(gate[t * gate_stride]) * shared[t][n]) (+ residual[t][n])
 * with scores == NULL meaning 1 (then out is gguf_experts kernel gguf_down's unweighted y, gguf_experts.py:499-526,
 * with T = n_slots, k = 1). Replaces gguf_down plus route_cuda.tail / the block's combine (route_cuda.py:256-264,
 * 291-298; stream_fast.py:4372-4376). h [T * k][I] fp32, shared [T][H] fp32 or NULL, gate fp32 or NULL,
 * residual [T][H] in rdtype or NULL, out [T][H] in odtype. ids >= n_experts contribute zero. */
int lmoe_gemv_down_combine(const float *h, const uint32_t *ids, const float *scores, int T, int k,
                           const uint8_t *wd, int type_d, int n_experts, int I, int H, const float *shared,
                           const float *gate, int gate_stride, const void *residual, int rdtype, void *out,
                           int odtype, void *stream);

/* The decode chain on rows of one slot each (topk 1), with weight reuse: rows go in windows of up to run_rows
 * (lowered to fit LDS), and a weight row is read once a run of equal consecutive slots in a window, so rows sorted
 * by slot read each expert once a window instead of once a row. Per row the arithmetic is the chain's (same
 * prepared units, unit dots and reduction tree), so h and out are meant to be bit-equal to lmoe_gemv_gate_up /
 * lmoe_gemv_down_combine (k 1, no scores); the Python layer checks that once a shape before using them. Replace
 * gguf_experts kernels gguf_gate_up_runs / gguf_down_runs (gguf_cuda.py:33-152) as driven by _gemv_runs
 * (gguf_experts.py:632-658). Q4_0 / Q4_K only; slots >= n_experts give zero rows.
 *   gate/up: x [n][H] in xdtype -> h [n][I] fp32;   down: h [n][I] fp32 -> out [n][H] in odtype, unweighted. */
int lmoe_gemv_gate_up_runs(const void *x, int xdtype, const uint32_t *slots, int n, int run_rows, const uint8_t *wg,
                           const uint8_t *wu, int type_g, int type_u, int n_experts, int H, int I, float *h,
                           void *stream);
int lmoe_gemv_down_runs(const float *h, const uint32_t *slots, int n, int run_rows, const uint8_t *wd, int type_d,
                        int n_experts, int I, int H, void *out, int odtype, void *stream);

/* The drop-in decode chain in its register-resident form (gguf_experts.gemv at one Q4 type for gate and up, a Q4
 * down, hidden 2048 or 4096, I a multiple of 128 up to 8192). Replace gguf_experts kernels gguf_gate_up and gguf_down
 * (gguf_experts.py:452-526) as driven by _chain (gguf_experts.py:610-629).
 *   gate/up: h[s] = silu(x[s / topk] . wg[slots[s]]) * (x[s / topk] . wu[slots[s]]) with x raw [n_slots / topk][H] in
 *            xdtype, prepared inside the launch (lmoe_prep_x's bits), the arithmetic of lmoe_gemv_gate_up_prepped;
 *            h [n_slots][I] fp32 and / or hprep [n_slots][I / 64 * 36] prepared for type_d without sums (either may
 *            be NULL);
 *   down:    out[s] = hprep[s] . wd[slots[s]], unweighted, [n][H] in odtype; each slot's units on an aligned group of
 *            16, 32 or 64 lanes with its own sum, so a slot's bits do not depend on the other slots of its call.
 * Slots >= n_experts give zero rows. */
int lmoe_gemv_chain_gate_up(const void *x, int xdtype, const uint32_t *slots, int n_slots, int topk, const uint8_t *wg,
                            const uint8_t *wu, int type, int n_experts, int H, int I, float *h, uint32_t *hprep,
                            int type_d, void *stream);
int lmoe_gemv_chain_down(const uint32_t *hprep, const uint32_t *slots, int n, const uint8_t *wd, int type_d,
                         int n_experts, int I, int H, void *out, int odtype, void *stream);

/* The run kernels for that chain: per row the arithmetic of lmoe_gemv_chain_gate_up / lmoe_gemv_chain_down (the same
 * staged rows, unit dots and cross-lane sums), so h, hprep and out are meant to be bit-equal to the chain's; the
 * Python layer checks that once a shape before using them. Replace gguf_gate_up_runs / gguf_down_runs
 * (gguf_cuda.py:33-152) as driven by _gemv_runs (gguf_experts.py:632-658).
 *   gate/up: x_prep [n][H / 64 * 36] (lmoe_prep_x for type) -> h [n][I] fp32 and / or hprep [n][I / 64 * 36];
 *   down:    hprep [n][I / 64 * 36] -> out [n][H] in odtype, unweighted.
 * Shapes and types as the chain's. Slots >= n_experts give zero rows. */
int lmoe_gemv_gate_up_runs_prepped(const uint32_t *x_prep, const uint32_t *slots, int n, int run_rows,
                                   const uint8_t *wg, const uint8_t *wu, int type, int n_experts, int H, int I,
                                   float *h, uint32_t *hprep, int type_d, void *stream);
int lmoe_gemv_down_runs_prepped(const uint32_t *hprep, const uint32_t *slots, int n, int run_rows, const uint8_t *wd,
                                int type_d, int n_experts, int I, int H, void *out, int odtype, void *stream);

/* lmoe_gemv_down_combine on h's prepared rows [T * k][I / 64 * 36] (has_sums 0: their half sums are derived from
 * the pairs, as lmoe_gemv_gate_up_prepped leaves them). type_d Q4_0 / Q4_K, Q6_K on rows prepared in the Q4_K
 * order (the 35B's down: one f16 rounding of h, v_dot2 on exact (q - 32) pairs) or Q8_0 on rows in the Q4_0 order
 * (v_dot2 on exact int8 pairs; experts 4-byte aligned). */
int lmoe_gemv_down_combine_prepped(const uint32_t *hprep, int has_sums, const uint32_t *ids, const float *scores,
                                   int T, int k, const uint8_t *wd, int type_d, int n_experts, int I, int H,
                                   const float *shared, const float *gate, int gate_stride, const void *residual,
                                   int rdtype, void *out, int odtype, void *stream);

/* Device-side ragged grouping: the stable counting sort of the flattened (token, k) expert ids, the device
 * form of stream_fast.py:5466-5471 (argsort of the flat ids and its inverse) and gguf_experts.py:702-713.
 * ids [R] -> counts [E], offsets [E + 1], order [R] (rows of expert 0 in flat order, then expert 1, ...; ids >= E
 * after all of them), inv [R] (inv[order[p]] = p), and the grouped GEMM's work list (tiles [max_tiles] of
 * (expert << 20 | first row / bm), n_tiles [1]) for m-tiles of bm rows. R <= 2^24, E <= 1024.
 * Workspace: lmoe_group_workspace_bytes(R, E). */
size_t lmoe_group_workspace_bytes(int R, int E);
int lmoe_group_rows(const uint32_t *ids, int R, int E, int bm, uint32_t *counts, uint32_t *offsets,
                    uint32_t *order, uint32_t *inv, uint32_t *tiles, uint32_t *n_tiles, void *ws, void *stream);
/* lmoe_group_rows with no workspace argument, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); no counterpart in the reference. The histograms
 * live in a file-scope device array of 1 MiB (lmoe_group_workspace_bytes(R, E) must not exceed it: R <= 519,936 at
 * E = 128, R <= 65,024 at E = 1024; larger requests are refused with LMOE_EWORKSPACE). The call
 * allocates nothing. Every call on one GPU shares that array, so calls that overlap on one GPU (two streams) race;
 * order them on one stream. Same arguments and results as lmoe_group_rows otherwise. */
int lmoe_group_rows_noalloc(const uint32_t *ids, int R, int E, int bm, uint32_t *counts, uint32_t *offsets,
                            uint32_t *order, uint32_t *inv, uint32_t *tiles, uint32_t *n_tiles, void *stream);
/* Upper bound on the grouped GEMM tiles for R rows over E experts at bm rows a tile. */
int lmoe_max_tiles(int R, int E, int bm);

/* Rows a grouped-GEMM m-tile covers: the bm that lmoe_group_rows and lmoe_max_tiles take for the grouped GEMMs. */
int lmoe_grouped_tile_rows(void);

/* The tuned launch choices for the grouped GEMMs, so every caller makes the same ones (no counterpart in the
 * reference, whose dense path has no tile size; gguf_experts.py:698-722 is the path they serve):
 * lmoe_grouped_pick_tile_rows: the grouping's bm for R rows over E experts with block types (type_g, type_u,
 *   type_d): 64 when gate/up runs on f16 weights (not Q4_0 / Q4_K, or gate and up of two types) or is Q4_K, 128
 *   for a Q4_0 gate/up with an f16 down, 32 when all three are Q4_0 and R < 16 E, else 128;
 * lmoe_grouped_pick_ksplit: split-K slices for one GEMM over K at that bm (4, 3 or 2 for 32-row tiles with
 *   R < 16 E, at least 4 K steps a slice; else 1);
 * lmoe_grouped_workspace_bytes: bytes of the ws that lmoe_grouped_gate_up_bm / lmoe_grouped_down_bm need with
 *   the picked ksplit of each (K = H for gate/up, I for down); 0 when neither splits. */
int lmoe_grouped_pick_tile_rows(int R, int E, int type_g, int type_u, int type_d);
int lmoe_grouped_pick_ksplit(int R, int E, int bm, int K);
size_t lmoe_grouped_workspace_bytes(int R, int E, int bm, int H, int I);

/* Grouped gate/up + SwiGLU on the matrix cores over rows grouped by lmoe_group_rows (bm = lmoe_grouped_tile_rows):
 *   h[p][f] = silu(x[order[p] / topk] . wg[e][f]) * (x[order[p] / topk] . wu[e][f])  for grouped row p of expert e,
 * h [R][I] float16 in grouped order (rows past offsets[E] untouched), each row in the GEMM K order (below).
 * x [T][H] float16 in the GEMM K order (xdtype must be LMOE_F16: lmoe_to_gemm_f16 makes it from any activation
 * dtype); wg / wu [E][I][row bytes], one ggml type (Q4_0 or Q4_K);
 * H a multiple of 64 (Q4_K: 256), I of 128. The work list is read on the device: max_tiles = lmoe_max_tiles(R, E,
 * bm). Replaces the reference's dense path dequant + gather_mm gate/up + silu-mul (gguf_experts.py:698-720;
 * DEQ_SRC :529-539). */
int lmoe_grouped_gate_up(const void *x, int xdtype, int T, int topk, const uint32_t *order, const uint32_t *offsets,
                         const uint32_t *tiles, const uint32_t *n_tiles, int max_tiles, const uint8_t *wg,
                         const uint8_t *wu, int type_g, int type_u, int n_experts, int H, int I, void *h,
                         void *stream);

/* Grouped down on the matrix cores: y[p][n] = h[p] . wd[e][n] for grouped row p of expert e, y [R][H] in ydtype
 * (F16 / F32) in grouped order, natural columns, unweighted. h [R][I] float16 in the GEMM K order, as
 * lmoe_grouped_gate_up leaves it; I a multiple of
 * 64 (Q4_K: 256), H of 256. Replaces the dense path's gather_mm down (gguf_experts.py:720-721). */
int lmoe_grouped_down(const void *h, const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles,
                      int max_tiles, const uint8_t *wd, int type_d, int n_experts, int I, int H, void *y, int ydtype,
                      void *stream);

/* lmoe_grouped_gate_up / lmoe_grouped_down over a grouping made with tile rows bm (lmoe_group_rows' bm): 128, or
 * 32 for Q4_0, whose 32-row tiles keep five K steps of weights in flight instead of three, for groups of few rows
 * (batched decode, prefill over many experts), where the GEMMs stream weights rather than reuse them. ksplit > 1
 * (32-row Q4_0 only; K / 64 divisible by it): split-K, ksplit workgroups a tile each taking a slice of K, their
 * fp32 sums in ws (16-byte aligned, ksplit * R * 2I floats for gate/up, ksplit * R * H for down; R = T * topk rows,
 * passed to down), then one finishing launch adds the slices in slice order and applies SwiGLU / the output
 * conversion: more workgroups when few tiles have work. No counterpart in the reference (its dense path has no
 * tile size). The entry points without bm use 128 and no split. */
int lmoe_grouped_gate_up_bm(const void *x, int xdtype, int T, int topk, const uint32_t *order,
                            const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles, int max_tiles,
                            int bm, int ksplit, float *ws, const uint8_t *wg, const uint8_t *wu, int type_g,
                            int type_u, int n_experts, int H, int I, void *h, void *stream);
int lmoe_grouped_down_bm(const void *h, int R, const uint32_t *offsets, const uint32_t *tiles,
                         const uint32_t *n_tiles, int max_tiles, int bm, int ksplit, float *ws, const uint8_t *wd,
                         int type_d, int n_experts, int I, int H, void *y, int ydtype, void *stream);

/* The stream layout of a Q4_0 / Q4_K expert matrix [n_experts][rows][row bytes] (no counterpart in the reference,
 * whose dense path reads the GGUF rows; it serves the same gather_mm, gguf_experts.py:698-722): the same bytes
 * ordered [expert][block of 128 features][K block] so that each grouped-GEMM step copies one contiguous run a block
 * of features. A K block is one 64-weight step for Q4_0 (4,608 bytes: the 128 features' 16-byte unit halves in the
 * GEMM's LDS order, then their 4-byte tails) and one super-block for Q4_K (18,432 bytes: the 128 headers, then four
 * steps of the features' 32-byte qs runs as 16-byte halves in the GEMM's LDS order). rows % 128 == 0.
 * lmoe_stream_bytes: its size (the GGUF matrix's), 0 for a type or shape without one; lmoe_stream_repack: writes
 * dst from the GGUF src (a one-time copy for a resident layer). */
size_t lmoe_stream_bytes(int type, int n_experts, int rows, int cols);
int lmoe_stream_repack(const uint8_t *src, int type, int n_experts, int rows, int cols, uint8_t *dst, void *stream);
/* lmoe_grouped_gate_up_bm / lmoe_grouped_down_bm on stream-layout weights (wg, wu, wd from lmoe_stream_repack),
 * bit-equal results; Q4_K at bm = 64 only. */
int lmoe_grouped_gate_up_sl(const void *x, int xdtype, int T, int topk, const uint32_t *order,
                            const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles, int max_tiles,
                            int bm, int ksplit, float *ws, const uint8_t *wg, const uint8_t *wu, int type_g,
                            int type_u, int n_experts, int H, int I, void *h, void *stream);
int lmoe_grouped_down_sl(const void *h, int R, const uint32_t *offsets, const uint32_t *tiles,
                         const uint32_t *n_tiles, int max_tiles, int bm, int ksplit, float *ws, const uint8_t *wd,
                         int type_d, int n_experts, int I, int H, void *y, int ydtype, void *stream);

/* lmoe_grouped_gate_up / lmoe_grouped_down with f16 weights in the K order (lmoe_dequant_gemm_f16's output:
 * wg16 / wu16 [n_experts][I][H], wd16 [n_experts][H][I]) instead of Q4 blocks: the grouped path of Q4_1, Q8_0,
 * Q5_K and Q6_K experts (the reference's gather_mm on dequantized f16 experts, gguf_experts.py:698-722). Same
 * grouping arguments, shapes (I % 128, H % 256 for down, K % 64) and outputs; bm: the grouping's tile rows, 128
 * or 64 (two workgroups a CU). */
int lmoe_grouped_gate_up_f16w(const void *x, int xdtype, int T, int topk, const uint32_t *order,
                              const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles, int max_tiles,
                              int bm, const void *wg16, const void *wu16, int n_experts, int H, int I, void *h,
                              void *stream);
int lmoe_grouped_down_f16w(const void *h, const uint32_t *offsets, const uint32_t *tiles, const uint32_t *n_tiles,
                           int max_tiles, int bm, const void *wd16, int n_experts, int I, int H, void *y, int ydtype,
                           void *stream);

/* The trunk's 4-bit affine matmul of T bf16 rows: out [T][N] bf16 = x [T][K] bf16 . W^T with W in MLX's
 * affine 4-bit layout (w uint32 [N][K / 8], element j of a word at bits 4j; scales, biases bf16 [N][K / G];
 * weight = q s + b), each row with the bits of the reference's route_cuda.qmv_rows (route_cuda.py:460-541; MLX
 * 0.32.4's one-row qmv): bf16 weights and bf16 fused multiply-add slots, float32 slot sum and lane butterfly.
 * K % 16 == 0, G % 16 == 0, K % G == 0; x 16-byte and w 8-byte aligned. */
int lmoe_qmv_rows(const void *x, int T, const uint32_t *w, const void *scales, const void *biases, int N, int K,
                  int group_size, void *out, void *stream);

/* out [n] bf16 = bf16(silu(g) u), float32 inside, one rounding: the SwiGLU of a shared expert run on
 * lmoe_qmv_rows projections (mlx_lm's nn.silu(gate) * up between the reference's qmv_rows calls; the reference
 * leaves it to MLX ops, whose bf16 bits are not reproduced here). */
int lmoe_swiglu_bf16(const void *g, const void *u, long long n, void *out, void *stream);

/* x [n] (F32 / BF16 / F16) -> out [n] float16, round to nearest even.
 * No counterpart in the reference (its dense path casts with MLX, gguf_experts.py:716). */
int lmoe_to_f16(const void *x, int xdtype, long long n, void *out, void *stream);

/* The grouped GEMMs' activation operand: x [n] (F32 / BF16 / F16, rows of a length divisible by 32, n % 32 == 0,
 * x and out 16-byte aligned) -> out [n] float16 (round to nearest even) in the GEMM K order: inside every 32-wide
 * block the elements run 0-3, 16-19, 4-7, 20-23, 8-11, 24-27, 12-15, 28-31. In that order each matrix-core lane's
 * 8 weights are the low and high nibbles of one 4-byte word of a Q4 block. No counterpart in the reference. */
int lmoe_to_gemm_f16(const void *x, int xdtype, long long n, void *out, void *stream);

/* Router logits of a prefill chunk on the matrix cores, replacing the reference's gate matmul before top-k
 * (stream_fast.py:4352-4360; route_cuda.py:433-444 on CUDA): xh [T][H] float16 in the GEMM K order (the activation
 * operand the grouped GEMMs read, lmoe_to_gemm_f16), wk [E + n_gate][H] float16 in the same order (the router
 * weight, plus the shared expert's gate row when n_gate == 1, converted once with lmoe_to_gemm_f16); exact f16
 * products, fp32 sums. logits [T][E] float32, gate [T] float32 (logit row E; null when n_gate == 0). H % 64 == 0.
 * lmoe_router_gemm_ksplit picks the K split (at least ~512 workgroups); with a split the partial sums go to ws
 * (lmoe_router_gemm_workspace_bytes, 16-byte aligned) and a second launch adds them in slice order. */
int lmoe_router_gemm_ksplit(int T, int H, int En);
size_t lmoe_router_gemm_workspace_bytes(int T, int H, int En);
int lmoe_router_gemm(const void *xh, int T, int H, const void *wk, int E, int n_gate, float *ws, float *logits,
                     float *gate, void *stream);

/* lmoe_router_gemm, then the top-k of its logits in the same pass over them (no counterpart in the reference; the
 * prefill router of stream_fast.py:4358-4370): ids / scores [T][k + m] as lmoe_router_topk (m == 0) or
 * lmoe_router_topk_shared (m > 0, n_gate == 1: slot k + j = (E + j, sigmoid(gate logit))) give them on the logits
 * lmoe_router_gemm writes, which are also written (logits, gate). With a K split, the top-k kernel adds the slices
 * itself, in lmoe_router_gemm's order: one launch fewer. E <= 1024, k <= 32, k + m <= 64. */
int lmoe_router_gemm_topk(const void *xh, int T, int H, const void *wk, int E, int n_gate, float *ws, float *logits,
                          float *gate, int k, int norm, int m, uint32_t *ids, float *scores, void *stream);

/* The prefill router's picks made exact (the prefill form of route_cuda.probs on the block's gate matmul,
 * stream_fast.py:4352-4370; the decode router's order, k_router_gemv, restated by the test oracle, fixes the bits).
 * lmoe_router_norms: norms [E (+1)][4] float32 of the router rows wr [E][H] (and the shared gate row wsg [H], when
 * given) in wdtype: |f16(w)|, |w|, |f16(w) - w|, |f16(w) restricted to f16 subnormals|, rounded up; once a layer.
 * lmoe_router_refine: from the router GEMM's logits M (part: its ksplit slices [ksplit][T][ldp], or the logits
 * [T][ldp] when ksplit == 1) and the raw x [T][H] in xdtype, each token's candidates are the experts whose M lies
 * within a proven bound of the k-th largest (the bound covers any summation order of the matrix cores, f16 rounding
 * of bf16 / f32 operands and flushed f16 subnormals); their logits are recomputed in the decode router's fixed order
 * (lmoe_router_gemv's bits), and ids / scores [T][k + m] are the top-k of those (ties to the lower index; slot k + j =
 * (E + j, sigmoid(gate logit)) when m > 0): the ids equal the decode router's on the same x, bit for bit. logits
 * [T][E] (optional, may alias part when ksplit == 1) receive the candidates' fixed-order logits and M elsewhere; gate
 * [T] (optional) the gate row's fixed-order logit; n_cand [T] (optional) the candidate counts. H % 8 == 0, H <= 8192,
 * E <= 1024, k <= 32, k + m <= 64, wr / wsg / norms 16-byte aligned. No counterpart in the reference.
 * lmoe_router_gemm_refine: lmoe_router_gemm (without its finish) then lmoe_router_refine on its slices; n_gate == 1
 * exactly when wsg is given (the GEMM then leaves the gate row out, since the refine recomputes it, but splits K as
 * for E + 1 rows; ws is sized by lmoe_router_gemm_workspace_bytes(T, H, E + n_gate) as before). ldp >= E. */
int lmoe_router_norms(const void *wr, const void *wsg, int wdtype, int E, int H, float *norms, void *stream);
int lmoe_router_refine(const float *part, int ksplit, int ldp, const void *x, int xdtype, int T, int H, const void *wr,
                       const void *wsg, int wdtype, int E, const float *norms, int k, int norm, int m, uint32_t *ids,
                       float *scores, float *logits, float *gate, int *n_cand, void *stream);
int lmoe_router_gemm_refine(const void *xh, int T, int H, const void *wk, int E, int n_gate, float *ws, const void *x,
                            int xdtype, const void *wr, const void *wsg, int wdtype, const float *norms, int k,
                            int norm, int m, uint32_t *ids, float *scores, float *logits, float *gate, int *n_cand,
                            void *stream);

/* Weighted combine of rows kept in grouped (expert-sorted) order:
 *   out[t][n] = sum_j scores[t][j] * y[inv[t * k + j]][n] (+ sigmoid(gate) * shared) (+ residual)
 * y [R][H] in ydtype. Replaces the unsort plus combine of stream_fast.py:5525 and 4372-4376. */
int lmoe_combine_sorted(const void *y, int ydtype, const uint32_t *inv, const float *scores, int T, int k, int H,
                        const float *shared, const float *gate, int gate_stride, const void *residual,
                        int rdtype, void *out, int odtype, void *stream);

/* Experts at `slots` of buf [S][rows][row bytes] as dense weights q [n][rows][cols] in odtype (F16, BF16, F32).
 * Replaces gguf_experts.dequant (gguf_experts.py:579-586; kernel gguf_dequant :529-539). */
int lmoe_dequant(const uint8_t *buf, int type, int n_experts, int rows, int cols, const uint32_t *slots, int n,
                 void *q, int odtype, void *stream);

/* Every expert of buf [n_experts][rows][row bytes] (any of the six types) as f16 weights out [n_experts][rows][cols]
 * in the grouped GEMMs' K order (within each 32 columns: 0-3, 16-19, 4-7, 20-23, 8-11, 24-27, 12-15, 28-31), the
 * operand of lmoe_grouped_*_f16w. The reference's prefill path dequantizes to f16 the same way before gather_mm
 * (gguf_experts.py:698-722, DEQ_SRC :529-539); cols % 32 (Q4_0/Q4_1/Q8_0) or % 256 (K types). */
int lmoe_dequant_gemm_f16(const uint8_t *buf, int type, int n_experts, int rows, int cols, void *out, void *stream);

/* Q4_0 quantizer on the device, ggml's quantize_row_q4_0_ref rule (no counterpart in the reference, which only
 * reads packs llama.cpp wrote): w [rows][cols] in wdtype -> out [rows][cols / 32 * 18]. */
int lmoe_quantize_q4_0(const void *w, int wdtype, long long rows, int cols, uint8_t *out, void *stream);

/* Q4_K quantizer on the device (no counterpart in the reference or in ggml): a plain min/scale fit, bit-for-bit the
 * CPU oracle's quantize_q4_k. w [rows][cols] in wdtype (cols % 256 == 0) -> out [rows][cols / 256 * 144]. Builds the
 * Q4_K test and benchmark packs (configuration 5). */
int lmoe_quantize_q4_k(const void *w, int wdtype, long long rows, int cols, uint8_t *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* LARDER_MOE_H */
