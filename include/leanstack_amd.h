/*
 * leanstack_amd.h - C ABI of the MI355X (gfx950) BF16 projection library.
 *
 * One shared library, libleanstack_amd.so, built with hipcc for gfx950 only.
 * It replaces the projection arithmetic of leanstack's Qwen3 semantic runtime:
 * the fused QKV, o_proj, fused gate_up with SiLU(gate)*up, down_proj and the
 * tied lm_head with its argmax, at M=1 (decode), M=2..16 (speculative verify)
 * and M in the thousands (prefill).
 *
 * Conventions
 *   - Plain pointers and sizes only.  Device pointers are HIP device memory
 *     owned by the caller; the library never allocates on the compute path.
 *   - Every compute entry point is asynchronous on `hip_stream` (a hipStream_t,
 *     NULL = the legacy default stream) and does no host synchronisation.
 *   - Return value: LSK_OK (0) or a negative lsk_status.  The message of the
 *     last failure on the calling thread is returned by lsk_last_error().
 *   - Argument checks run before anything touches the GPU, so a rejected call
 *     launches nothing.
 *
 * Weight layout LSK_LAYOUT_MFMA16X32 (the packed, resident layout)
 *   W[N][K] bf16 (N % 16 == 0, K % 32 == 0) is stored as N/16 row-blocks of
 *   K/32 tiles of 1024 bytes each, tile (rb, kt) at byte offset
 *   (rb * (K/32) + kt) * 1024.  Inside a tile, the 16 bytes at offset 16*l
 *   hold W[16*rb + l%16][32*kt + 8*(l/16) + e], e = 0..7: lane l of a
 *   64-wide wavefront loads the A operand of one v_mfma_f32_16x16x32_bf16
 *   with one 16-byte load.
 * Weight layout LSK_LAYOUT_MFMA16X32_GATEUP
 *   The same tiling applied to a fused [gate; up] matrix (N = 2*I) whose
 *   row-blocks are interleaved: packed row-block 2j holds gate rows
 *   16j..16j+15 and packed row-block 2j+1 holds up rows 16j..16j+15, so the
 *   SiLU(gate)*up epilogue reads both halves from the same lanes.
 */
#ifndef LEANSTACK_AMD_H
#define LEANSTACK_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LSK_ABI_VERSION 3

enum lsk_layout {
  LSK_LAYOUT_ROWMAJOR = 0,        /* plain W[N][K]; accepted by the packer only */
  LSK_LAYOUT_MFMA16X32 = 1,       /* 1 KB MFMA A-operand tiles (see above) */
  LSK_LAYOUT_MFMA16X32_GATEUP = 2 /* same tiles, gate/up row-blocks interleaved */
};

enum lsk_epilogue {
  LSK_EPI_NONE = 0,         /* y = bf16(x . W^T) */
  LSK_EPI_SILU_MUL = 1,     /* y = bf16(bf16(silu(bf16(g))) * bf16(u)), [g|u] = x . W^T */
  LSK_EPI_RESIDUAL_ADD = 2  /* y = bf16(residual + bf16(x . W^T)) */
};

enum lsk_op {
  LSK_OP_LINEAR = 0,
  LSK_OP_LM_HEAD_ARGMAX = 1
};

enum lsk_logits_mode {
  LSK_LOGITS_FP32 = 0,  /* argmax over fp32 scores (cuTile head semantics) */
  LSK_LOGITS_BF16 = 1   /* argmax over bf16-rounded logits (torch.mv head semantics) */
};

enum lsk_status {
  LSK_OK = 0,
  LSK_ERR_INVALID = -1,    /* bad shape, stride, alignment, M or epilogue */
  LSK_ERR_LAYOUT = -2,     /* unknown or unsupported weight layout id */
  LSK_ERR_HIP = -3,        /* a HIP runtime call or kernel launch failed */
  LSK_ERR_WORKSPACE = -4   /* workspace missing or smaller than lsk_workspace_bytes() */
};

/* ABI version of the loaded library (LSK_ABI_VERSION it was built with). */
int lsk_abi_version(void);

/* Message of the last failed call on this thread ("" if none).  Valid until
 * the next call into the library from the same thread. */
const char* lsk_last_error(void);

/* Bytes of one packed weight matrix W[N][K] in `layout_id`; 0 if the shape or
 * layout is not supported.  Replaces the per-tensor size accounting of
 * leanstack's packer (src/leanstack/pack.py:190-209). */
size_t lsk_packed_bytes(int layout_id, int N, int K);

/* Device workspace that `op` needs for M rows of an [N, K] weight.  The
 * caller allocates it once and passes it to every call of that op.  For
 * LSK_OP_LM_HEAD_ARGMAX it is required; it replaces the tile_scores /
 * tile_argmax scratch that src/leanstack/runtime/cutile_logits.py:56-58
 * allocates per call.  For LSK_OP_LINEAR it is optional and sized for the
 * current device's CU count (0 when the shape does not use one). */
size_t lsk_workspace_bytes(int op, int M, int N, int K);

/* Host-side packer: re-tile row-major W[N][K] bf16 (`w_rowmajor_host`) into
 * `layout_id` at `out_host` (lsk_packed_bytes() bytes).  For
 * LSK_LAYOUT_MFMA16X32_GATEUP the input is the fused [gate; up] matrix with
 * gate rows first, as leanstack's packer concatenates it
 * (src/leanstack/pack.py:281-284).  Replaces the row-major fusion of
 * src/leanstack/pack.py:269-286. */
int lsk_pack_bf16(const void* w_rowmajor_host, int N, int K, int layout_id, void* out_host);

/* Inverse of lsk_pack_bf16 (out_rowmajor_host receives W[N][K]). */
int lsk_unpack_bf16(const void* packed_host, int N, int K, int layout_id, void* out_rowmajor_host);

/* How lsk_linear_bf16 runs M rows of an [N, K] weight on the current device
 * with a workspace of ws_bytes (0: none).
 *   17 <= M <= 64, and 65 <= M <= 128 unless N >= 8192 is on the 128-row
 *   GEMM grid (the skinny kernel; N % 16 == 0, K % 32 == 0): plan[0] =
 *   weight rows per workgroup (16, 32 or 64), plan[1] = N / plan[0] row
 *   groups, plan[2] = the groups whose K range is split (all or none),
 *   plan[3] = workgroups per group (1: no split).  This is the plan of the
 *   plain and residual epilogues; a SiLU*up call takes whole gate/up pairs
 *   (32 or 64 rows) and may split differently.
 *   M > 128: plan[0] = weight rows per output block of the prefill block GEMM
 *   (256, 192 or 128), plan[1] = output blocks, plan[2] = blocks whose K
 *   range is split over several workgroups, plan[3] = workgroups (K chunks)
 *   per split block (1: no split).
 * plan = {0, 0, 0, 1} whenever the call takes none of those: the decode
 * kernels (M <= 16, or M > 128 with N or K off every GEMM tile grid), the
 * 256x256 GEMM with both operands staged in LDS (M > 128, N % 256 == 0,
 * K % 64 == 0 but not a shape the block GEMM takes, e.g. K an odd multiple of
 * 64) or the 128x128 GEMM (65 <= M <= 128 with N >= 8192, and the rest of
 * M > 128 with N % 128 == 0, K % 64 == 0).  A workspace smaller than
 * lsk_workspace_bytes(LSK_OP_LINEAR, M, N, K) is refused with
 * LSK_ERR_WORKSPACE, as lsk_linear_bf16 refuses it.  For tests and tuning; no
 * counterpart in the reference, whose F.linear hides its cuBLAS plan. */
int lsk_linear_plan(int M, int N, int K, size_t ws_bytes, int plan[4]);

/* y[M][*] = epilogue(x[M][K] . W[N][K]^T), bf16 in and out, fp32 accumulate.
 *   w_packed   device, layout LSK_LAYOUT_MFMA16X32 (epilogue NONE / RESIDUAL_ADD)
 *              or LSK_LAYOUT_MFMA16X32_GATEUP (epilogue SILU_MUL; N = 2*I)
 *   x          device bf16, row m at x + m*ldx (ldx >= K, ldx % 8 == 0,
 *              ldx <= 2^22 - 8, 16-byte aligned)
 *   y          device bf16, row m at y + m*ldy; N columns, or N/2 for
 *              SILU_MUL (ldy % 4 == 0, 8-byte aligned)
 *   residual   device bf16 [M][N] at stride ldr, RESIDUAL_ADD only (else NULL)
 *   M          >= 1.  M <= 16 runs the decode/verify kernel (weights streamed
 *              once, activations padded to the 16 MFMA columns); 17..128 the
 *              skinny kernel (weights streamed once, activations in groups
 *              of 16 tokens; 65..128 rows of N >= 8192 the 128x128 GEMM);
 *              larger M the prefill MFMA GEMM.
 *   workspace  NULL, or lsk_workspace_bytes(LSK_OP_LINEAR, M, N, K) bytes
 *              (0 bytes: no workspace is used), 256-byte aligned, zero-filled
 *              before its first use.  With it, the prefill GEMM splits the K
 *              range of the output blocks of its last, partial round over the
 *              idle CUs (split-K), and the skinny kernel splits the K range
 *              of every row-block when the row-blocks alone leave CUs idle;
 *              both add the fp32 partials in a fixed order.  Without it, one
 *              workgroup per output block.  Calls leave it as they found it
 *              (see lsk_linear_error); calls that share one must be
 *              stream-ordered.  Ignored for M <= 16.
 * Replaces torch.mv / F.linear at src/leanstack/runtime/qwen_explicit.py:748,
 * :787, :819, :828-830, :913, :942-948, :1202-1208. */
int lsk_linear_bf16(const void* w_packed, int layout_id, int N, int K,
                    const void* x, int M, int ldx,
                    void* y, int ldy,
                    int epilogue, const void* residual, int ldr,
                    void* workspace, size_t ws_bytes, void* hip_stream);

/* y[M][*] = epilogue(rms_norm(x)[M][K] . W[N][K]^T) for M = 1..16, with
 *   rms_norm(x)[m][k] = bf16((x[m][k] * r[m]) * norm_weight[k]),
 *   r[m] = 1 / sqrt(sum_k x[m][k]^2 / K + eps), fp32 arithmetic,
 * the RMSNorm computed inside the projection kernel (no normalised copy of x
 * is written).  Arguments as for lsk_linear_bf16 (workspace: none), plus
 *   norm_weight  device bf16 [K], 16-byte aligned
 *   eps          finite, >= 0
 * Replaces the F.rms_norm in front of the decode / verify QKV and gate_up
 * projections: qwen_rmsnorm_vector + torch.mv at
 * src/leanstack/runtime/qwen_explicit.py:1255 (input_layernorm, then QKV at
 * :787) and :941-942 (post_attention_layernorm, then gate_up), and
 * F.rms_norm + F.linear at :821-827 for the verify rows. */
int lsk_rmsnorm_linear_bf16(const void* w_packed, int layout_id, int N, int K,
                            const void* x, int M, int ldx,
                            const void* norm_weight, float eps,
                            void* y, int ldy,
                            int epilogue, const void* residual, int ldr,
                            void* hip_stream);

/* Device workspace of lsk_decode_attention_bf16 for n_kv kv heads of
 * n_q / n_kv q heads and caches of max_seq_len rows (0 if the geometry is not
 * supported).  Needed once more than 128 rows are attended. */
size_t lsk_attention_workspace_bytes(int n_q, int n_kv, int head_dim, int max_seq_len);

/* One decode token of one layer, between its QKV and o_proj projections:
 *   q heads and k heads of `qkv` (the raw QKV projection row [n_q*d | n_kv*d |
 *   n_kv*d], bf16) get the per-head RMSNorm over d with q_norm_weight /
 *   k_norm_weight and eps, then rotate-half RoPE with `cos` / `sin` (bf16
 *   [d/2], this position's row of the position cache), with a bf16 rounding
 *   after each step as the reference's torch ops round;
 *   k and v are written to row `pos` of k_cache / v_cache (this layer's
 *   [n_kv][max_seq_len][d] bf16, 16-byte aligned);
 *   out[n_q*d] = softmax(q K^T * scale) V over rows 0..pos, q head h reading
 *   kv head h / (n_q/n_kv), fp32 scores and softmax, bf16 output.
 * d must be 128, n_kv at most 64, n_q/n_kv one of 1, 2, 4, 8, and
 * max_seq_len at most 16384.  The pos+1 rows run as one chunk up to 128
 * rows, as at most 8 chunks of 64 rows up to 512 rows, and beyond that as at
 * most 32 chunks of 128, 256, 384 or 512 rows (the smallest that fits), one
 * workgroup each; with more than one chunk the partial results meet in
 * `workspace` (lsk_attention_workspace_bytes(), 256-byte aligned,
 * zero-filled before its first use; calls leave it zeroed; calls sharing one
 * must be stream-ordered), combined in chunk order so results are bitwise
 * reproducible.  With up to 128 rows the workspace may be NULL.  The caller
 * advances its sequence length.  Replaces the per-head norms and RoPE of
 * src/leanstack/runtime/qwen_explicit.py:796-806 (RoPE :690-716), the cache
 * append of src/leanstack/runtime/kv_cache.py:222-245 and the
 * F.scaled_dot_product_attention of qwen_explicit.py:894-912. */
int lsk_decode_attention_bf16(const void* qkv, int n_q, int n_kv, int head_dim,
                              const void* q_norm_weight, const void* k_norm_weight, float eps,
                              const void* cos, const void* sin,
                              void* k_cache, void* v_cache, int max_seq_len, int pos,
                              float scale, void* out,
                              void* workspace, size_t ws_bytes, void* hip_stream);

/* The same step with the position in device memory, for a decode step
 * captured once as a HIP graph and replayed for every token (the caller
 * writes the next position into *pos_device between replays): cos_table /
 * sin_table are the whole position tables [max_seq_len][d/2] (bf16, the
 * reference's position cache, src/leanstack/runtime/qwen_explicit.py:664-676),
 * of which row *pos_device is used.  The launch shape does not depend on the
 * position, so the workspace is required once max_seq_len exceeds 128.  A
 * *pos_device outside [0, max_seq_len) leaves every buffer untouched.  Same
 * results as lsk_decode_attention_bf16 at that position, bit for bit.
 * Replaces the same reference code as lsk_decode_attention_bf16. */
int lsk_decode_attention_at_bf16(const void* qkv, int n_q, int n_kv, int head_dim,
                                 const void* q_norm_weight, const void* k_norm_weight, float eps,
                                 const void* cos_table, const void* sin_table,
                                 void* k_cache, void* v_cache, int max_seq_len, const int* pos_device,
                                 float scale, void* out, void* workspace, size_t ws_bytes,
                                 void* hip_stream);

/* Greedy lm_head: out_idx[m] = argmax_v sum_k f32(W[v][k]) * f32(x[m][k]) for
 * m < M (M = 1..16), lowest index on ties.  V % 16 == 0 (whole packed
 * row-blocks; a tensor-parallel vocab shard, e.g. 151936 / 8 = 18992, has an
 * odd count of them), K % 32 == 0.
 *   logits_mode  LSK_LOGITS_FP32 compares fp32 scores, as the cuTile kernel
 *                does (src/leanstack/runtime/cutile_logits.py:17-31, :67-69);
 *                LSK_LOGITS_BF16 compares bf16-rounded logits, as
 *                torch.mv(...).argmax does
 *                (src/leanstack/runtime/qwen_explicit.py:952-960).
 *   logits_opt   NULL, or device fp32 [M][V] that receives the scores.
 *   out_idx      device int64 [M].
 *   workspace    lsk_workspace_bytes(LSK_OP_LM_HEAD_ARGMAX, M, V, K) bytes,
 *                8-byte aligned, ZERO-FILLED before its first use (e.g.
 *                hipMemset(ws, 0, bytes)); every call leaves it zero again,
 *                so one zeroing serves every later call.  Calls that share a
 *                workspace must be stream-ordered.  Its first word counts
 *                argmax stages that gave up waiting for a partial (then
 *                that row's out_idx is -1); it stays 0 while the grid runs
 *                to completion.
 * One launch: the workgroups store per-tile maxima and the last M
 * workgroups of the grid reduce them.
 * Replaces cutile_logits_argmax (src/leanstack/runtime/cutile_logits.py:37-69)
 * and the per-position head loop of the verify path
 * (experiments/models/qwen_explicit_runtime_loop.py:805-812) with one M-row
 * call. */
int lsk_lm_head_argmax_bf16(const void* w_packed, int layout_id, int V, int K,
                            const void* x, int M, int ldx,
                            float* logits_opt, int logits_mode,
                            long long* out_idx,
                            void* workspace, size_t ws_bytes, void* hip_stream);

/* The same with the final RMSNorm of x applied in the kernel (norm_weight
 * [K] bf16, 16-byte aligned; eps): out_idx = argmax(rms_norm(x) . E^T), with
 * each normalised value bf16(x*w*r) as in lsk_rmsnorm_linear_bf16.  K must
 * be 2560 (the Qwen3-4B hidden size) and M at most 8.  Replaces the final
 * norm and head of src/leanstack/runtime/qwen_explicit.py:952-960 (and,
 * with LSK_LOGITS_FP32, the norm in front of cutile_logits_argmax,
 * qwen_explicit.py:1807-1832) in the same one launch. */
int lsk_rmsnorm_lm_head_argmax_bf16(const void* w_packed, int layout_id, int V, int K,
                                    const void* x, int M, int ldx,
                                    const void* norm_weight, float eps,
                                    float* logits_opt, int logits_mode, long long* out_idx,
                                    void* workspace, size_t ws_bytes, void* hip_stream);

/* lsk_lm_head_argmax_bf16 without the workspace: the argmax workspace lives
 * in a static device array of the library (1 MiB per device, zero from load
 * time), so the call allocates nothing.  No counterpart in the reference; it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Limit:
 * 64 + M * P * 8 bytes must fit in 1 MiB, P the scoring workgroups: with
 * NB = V/16 row-blocks, P = NB up to 512 of them, else (NB - T)/2 + T with
 * T = 512 + (NB - 512) % 2 (every M <= 16 at V = 151936, P = 5004); larger
 * calls return LSK_ERR_INVALID before anything touches the GPU.  All calls on one
 * device share the array: calls that overlap in time on a device (streams not
 * ordered with each other) race; stream-ordered calls do not. */
int lsk_lm_head_argmax_noalloc_bf16(const void* w_packed, int layout_id, int V, int K,
                                    const void* x, int M, int ldx,
                                    float* logits_opt, int logits_mode, long long* out_idx,
                                    void* hip_stream);

/* ------------------------------------------------------------------------
 * Stack programs: a whole decode / verify step of projections in ONE launch.
 *
 * A program is a list of projections with the semantics of lsk_linear_bf16
 * (all at the same M = 1..16 rows) plus a dependency per projection.  The
 * persistent kernel streams the weights of every projection in order and
 * starts loading a projection's weights before its input is ready; only the
 * multiply waits.  This replaces the per-layer Python loop of
 * run_semantic_stack_decode (src/leanstack/runtime/qwen_explicit.py:1636-1643)
 * and its 4 projection launches per layer.
 * ------------------------------------------------------------------------ */

typedef struct lsk_projection {
  const void* w_packed;  /* packed weights, as for lsk_linear_bf16 */
  int layout_id;
  int N;
  int K;                 /* a multiple of 512 */
  const void* x;         /* input rows [M][K] at stride ldx */
  int ldx;
  void* y;               /* output rows at stride ldy */
  int ldy;
  int epilogue;          /* lsk_epilogue */
  const void* residual;  /* RESIDUAL_ADD only, else NULL */
  int ldr;
  int depends_on;        /* -1: inputs ready at launch; q (< this index):
                            every projection 0..q finishes before this one
                            reads x or residual */
} lsk_projection;

/* Device bytes of a program of `count` projections. */
size_t lsk_stack_program_bytes(int count);

/* Device workspace bytes of a program of `count` projections (an error word,
 * the detail record of the first failed wait and one progress word per CU;
 * 8 KiB).  The caller zeroes it once before the first launch; every launch
 * leaves its synchronisation words zeroed again (the error word aside, see
 * lsk_stack_error). */
size_t lsk_stack_workspace_bytes(int count);

/* Validate `projections` (host array, count = 1..256) and upload the program to
 * program_dev (device, lsk_stack_program_bytes(count) bytes).  Synchronous;
 * set-up only. */
int lsk_stack_prepare(const lsk_projection* projections, int count, int M, void* program_dev,
                      size_t program_bytes);

/* Launch a prepared program on hip_stream (one kernel; capturable in a HIP
 * graph).  No other kernel may run on the device concurrently: the program
 * keeps one workgroup resident per CU.  Launches that share a workspace must
 * be stream-ordered. */
int lsk_stack_run(const void* program_dev, int count, void* workspace, size_t ws_bytes, void* hip_stream);

/* Read (synchronously) and clear the workspace's error word: 0 = every wait
 * of every launch since the last call completed; nonzero = a bounded wait
 * gave up (outputs of that launch are invalid). */
int lsk_stack_error(void* workspace, int* error_out);

/* Read (synchronously) and clear the error word of a prefill workspace:
 * 0 = every wait of every split-K launch since the last call completed;
 * nonzero = a bounded wait for another workgroup's partial gave up (outputs
 * of that launch are invalid).  No counterpart in the reference, whose
 * library GEMMs have no cross-workgroup waits. */
int lsk_linear_error(void* workspace, int* error_out);

/* Polls of a split-K arrival word before a prefill workgroup stops waiting
 * for the other chunks of its output block (default 4194304, about 0.1 s).
 * A workgroup that gives up sets the workspace's error word (see
 * lsk_linear_error) and writes NaN to its share of the block, so a lost wait
 * is never returned as a result.  Applies to launches after the call; used
 * by tests to force the give-up path from the host.  No counterpart in the
 * reference, whose library GEMMs have no cross-workgroup waits. */
void lsk_set_linear_wait_limit(unsigned polls);

/* Kernel-duration measurement for benchmarks.  Between
 * lsk_dispatch_timing_begin and lsk_dispatch_timing_end on one host thread,
 * each kernel the library launches from that thread (up to max_dispatches,
 * 1..65536) carries a start/stop event pair bound to the dispatch itself, so
 * the elapsed time is the kernel's own execution time, as a profiler's
 * kernel trace measures it (no launch gaps).  end waits for those events,
 * writes the duration in microseconds of the first min(capacity, n) timed
 * dispatches, in launch order, to durations_us (host) and n to *dispatches
 * (launches past max_dispatches run untimed).  Not for launches into a
 * stream that is being captured.  No counterpart in the reference, whose
 * benchmarks time with torch CUDA events around whole calls. */
int lsk_dispatch_timing_begin(int max_dispatches);
int lsk_dispatch_timing_end(float* durations_us, int capacity, int* dispatches);

/* Measurement of what a single-launch decode step could reach (bench.py
 * --probe-step-floor).  One persistent workgroup per CU streams `count`
 * segments of 1 KB tiles from `weights` (sum(seg_tiles) * 1024 bytes, any
 * contents; each seg_tiles[s], host, a multiple of the CU count and at
 * least 12 per CU)
 * through 12 compute waves holding `ring` (4 or 16) tile loads each in
 * flight, every CU taking an equal contiguous share of each segment and
 * multiplying every tile.  mode 0: no dependency between segments; mode 1:
 * before the first multiply of segment s + 1 every workgroup waits until all
 * have finished segment s, on one arrival word per segment; mode 2: the same
 * on a two-level barrier (8 group words, the last arrival of each group
 * counts globally and releases its group); mode 3: the same on tag words
 * (every workgroup stores s + 1 into its word of 8 replicas of a tag array
 * and polls its replica until every word has reached it; at most 256 CUs).
 * The weight loads run ahead across the waits.  workspace: lsk_probe_workspace_bytes() bytes,
 * zero-filled before first use; every launch leaves it zero except word 0,
 * which is nonzero after a bounded wait gave up.  No counterpart in the
 * reference. */
size_t lsk_probe_workspace_bytes(void);
/* Measurement of the dense BF16 MFMA rate (bench.py --probe-mfma): each of
 * `workgroups` workgroups of 4 waves runs `iterations` x 64
 * v_mfma_f32_32x32x16_bf16 (16 accumulator tiles per wave, operands in
 * registers, 32768 FLOP each), with no memory traffic.  sink: one device
 * word, written only if a checksum takes a value it never takes.  No
 * counterpart in the reference. */
int lsk_probe_mfma_rate(int workgroups, int iterations, void* sink, void* hip_stream);
int lsk_probe_stream_step(const void* weights, size_t weight_bytes, const long long* seg_tiles, int count, int mode,
                          int ring, void* workspace, size_t ws_bytes, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* LEANSTACK_AMD_H */
