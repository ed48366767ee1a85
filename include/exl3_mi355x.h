/* C-ABI of the MI355X (gfx950) EXL3 hot-path library, libexl3_mi355x.so.
 *
 * Conventions (the reference's, cuda/csrc/exl3_marlin.cu:411-535, restated for a C boundary):
 *   - every pointer argument is DEVICE memory unless named *_host; tensors are contiguous, row-major;
 *   - fp16 / bf16 values are passed as raw 16-bit storage; `*_bf16` flags pick bf16 over fp16 at the boundary,
 *     with torch's value conversions (bf16 -> fp16 round-to-nearest-even, overflow to inf; fp16 -> bf16 RNE);
 *   - `stream` is a hipStream_t (NULL = the default stream); every call only enqueues work (no host sync,
 *     no allocation); the caller owns every buffer, including `workspace`;
 *   - each call returns EXL3_OK or an error code; exl3_last_error() then holds a message (thread-local).
 *     Where the reference raised (TORCH_CHECK -> RuntimeError), this library returns EXL3_ERR_INVALID and
 *     launches nothing.
 *   - a call with zero rows (tokens, slots, sequences) launches nothing and returns EXL3_OK once its other
 *     arguments check out; its activation, output and routing pointers may then be NULL (weights, sign vectors
 *     and caches are still checked).
 *
 * The EXL3 format (core/src/trellis_core/format/spec.py:117-160): trellis int16 [k/16, n/16, 16K], K bits per
 * weight in {2,3,4,5,6,8}, k and n multiples of 128; suh fp16 [k], svh fp16 [n]; codebook 0 = 3INST, 1 = MCG,
 * 2 = MUL1 (core/src/trellis_core/reference.py:24-77).
 */
#ifndef EXL3_MI355X_H
#define EXL3_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_ABI_VERSION 6

enum {
  EXL3_OK = 0,
  EXL3_ERR_INVALID = 1,     /* bad shape / argument; nothing was launched */
  EXL3_ERR_HIP = 2,         /* a HIP runtime call failed */
  EXL3_ERR_UNSUPPORTED = 3  /* valid request this build does not serve (e.g. not a gfx950 device) */
};

#define EXL3_MAX_SHARDS 4

/* The first EXL3_WORKSPACE_COUNTER_BYTES of every exl3_linear / exl3_gemm_rotated / exl3_moe_forward workspace hold
 * the split counters (one int per output column block).  They must be zero before the first call on a workspace;
 * every call leaves them zero again, so calls of any shapes may share one workspace (ordered on one stream).  The
 * region sits at a fixed place so that no call reads another call's partials as counters. */
#define EXL3_WORKSPACE_COUNTER_BYTES (256u * 1024u)

/* One matrix of a fused group (q/k/v, gate/up): all shards read the same input x and write adjacent column spans
 * of y in order.  Replaces the per-shard tensors of exl3_linear_marlin_multi_out (cuda/csrc/exl3_marlin.cu:507-527)
 * and the shard map of the Marlin template (exl3_marlin_template.h:298-302, 605-610). */
typedef struct exl3_shard {
  const void* trellis; /* the trellis in `layout`: the stored int16 [k/16, n/16, 16K], or exl3_repack_trellis's */
  const void* suh;     /* fp16 [k] */
  const void* svh;     /* fp16 [n] */
  int n;               /* output columns of this shard (multiple of 128) */
  int layout;          /* EXL3_LAYOUT_STORED (0, zero-initialised callers) or EXL3_LAYOUT_BLOCKS */
} exl3_shard;

/* Trellis layouts.  STORED: the checkpoint's int16 [k/16, n/16, 16K], tile (i, j) at byte (i n/16 + j) 32K.
 * BLOCKS: the load-time layout of exl3_repack_trellis, the same tiles reordered so that each (128-column block cb,
 * 128-row block kb) unit of 8 x 8 tiles is one contiguous 2048K-byte run, units column block major, and inside a
 * unit the 8 tiles of each tile column contiguous: tile (i, j) at byte
 * ((j / 8) (k / 128) + i / 8) 2048K + ((j % 8) 8 + i % 8) 32K.  Same bytes per tile, lossless. */
#define EXL3_LAYOUT_STORED 0
#define EXL3_LAYOUT_BLOCKS 1

/* ---- process / device ---------------------------------------------------------------------------------------- */
int exl3_abi_version(void);
const char* exl3_last_error(void);
/* Checks that `device` is a gfx950, then probes (one small launch, synchronous) that workgroups whose ids agree mod 8
 * run on one XCD; once a probe has passed, decode-GEMV launches whose column-block count is a multiple of 8 keep their
 * split-K partials and counters in that XCD's L2 (otherwise, and before any call here, they use device-coherent
 * accesses; results are the same bits either way).  Call it before capturing graphs.  Replaces init_device
 * (cuda/csrc/exl3_marlin.cu:537). */
int exl3_init_device(int device);
/* 1 when split-K chains may stay in one XCD's L2 (a probe of exl3_init_device passed and EXL3_GEMV_XCD_LOCAL is not
 * 0), else 0.  No counterpart in the reference: it reports which chain the launches of this process use. */
int exl3_xcd_local_chains(void);

/* ---- decode (subsystem 1) ------------------------------------------------------------------------------------- */
/* W_inner fp16 [k, n] = the decoded trellis (Hadamard domain, no sign vectors), bit-identical to
 * trellis_core.reference.reconstruct_inner (core/src/trellis_core/reference.py:102-115).  Replaces ExLlamaV3's
 * `reconstruct` as called at cuda/src/sglang_exl3/kernels/reference.py:71-76 and xpu/csrc/exl3_ops.sycl:536. */
int exl3_reconstruct(const void* trellis, int k, int n, int K, int codebook, void* w_out, void* stream);
/* Load-time repack of a stored trellis int16 [k/16][n/16][16K] (k, n multiples of 128) into EXL3_LAYOUT_BLOCKS
 * (k*n*K/8 bytes, a permutation of whole tiles; out must not alias the input; both 16-byte aligned).  Lossless;
 * exl3_unpack_trellis inverts it bit for bit.  exl3_linear, exl3_linear_noalloc and exl3_linear_prefill read a
 * repacked shard when its `layout` says so (same results); exl3_reconstruct, exl3_gemm_rotated and the MoE entry
 * points read the stored layout.  Replaces repack_trellis (cuda/csrc/exl3_marlin.cu:344-381, called by prepare,
 * cuda/src/sglang_exl3/kernels/marlin.py:65-76). */
int exl3_repack_trellis(const void* trellis, int k, int n, int K, void* out, void* stream);
/* Inverse of exl3_repack_trellis: the stored layout back.  Replaces unpack_trellis (exl3_marlin.cu:384-408). */
int exl3_unpack_trellis(const void* packed, int k, int n, int K, void* out, void* stream);

/* ---- Hadamard rotations (subsystem 4) ------------------------------------------------------------------------- */
/* xh[s*rows + r, :] = fp16(Had128(fp16(x[r, :]) * suh_cat[s, :])) for shards s < shards; xh fp16 [shards*rows, k].
 * Replaces had_in_group_marlin (cuda/csrc/exl3_marlin.cu:461-471). */
int exl3_had_in_group(const void* x, int x_bf16, int rows, int k, const void* suh_cat, int shards, void* xh,
                      void* stream);
/* out[r, col0 : col0+n] = fp16(Had128(y[r, :])) * svh, stored fp16 or bf16 with row stride ld_out (elements).
 * y fp16 [rows, n].  Replaces had_out_into_marlin (cuda/csrc/exl3_marlin.cu:475-484). */
int exl3_had_out_into(const void* y, int rows, int n, const void* svh, void* out, int out_bf16, int ld_out, int col0,
                      void* stream);

/* ---- fused decode-GEMV / GEMM (subsystems 2, 3) --------------------------------------------------------------- */
/* Workspace bytes exl3_linear needs for `rows` rows of a group with input width k and `n_total` output columns
 * (n_total / 128 at most EXL3_WORKSPACE_COUNTER_BYTES / 4); 0 means none.  Deterministic in its arguments.  The
 * workspace holds the split counters (EXL3_WORKSPACE_COUNTER_BYTES, zero before the first use) and fp32 split
 * partials; calls that share a workspace must be ordered on one stream.  exl3_linear checks the workspace against the
 * split plans of its own launches and returns EXL3_ERR_INVALID, launching nothing, when it is short. */
size_t exl3_linear_workspace_bytes(int rows, int k, int n_total, int K);

/* y[rows, sum n_s] = concat_s( Had128(Had128(x * suh_s) @ W_s) * svh_s ) with fp32 accumulation; fp16 output of
 * the GEMM, output transform as exl3_had_out_into.  x fp16|bf16 [rows, k]; y fp16|bf16 [rows, sum n_s].
 * All shards share K and codebook.  One launch serves up to 64 rows (each decoded tile feeds 1, 2 or 4 16-row MFMA
 * groups); more rows take more launches.  Replaces exl3_linear_marlin_out / exl3_linear_marlin_multi_out
 * (cuda/csrc/exl3_marlin.cu:489-527) behind torch.ops.sglang_exl3.linear (cuda/src/sglang_exl3/runtime/ops.py:133). */
int exl3_linear(const void* x, int x_bf16, int rows, int k, const exl3_shard* shards_host, int nshards, int K,
                int codebook, void* y, int y_bf16, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of exl3_gemm_rotated for `rows` rows (below 65 rows those of its decode-GEMV launches, from 65 rows
 * those of the prefill decode-GEMM); 0 for bad shapes.  Same counter-region contract as exl3_linear_workspace_bytes. */
size_t exl3_gemm_rotated_workspace_bytes(int rows, int k, int n, int K);
/* out fp16 [rows, n] = xh @ W_inner in the rotated basis (no Hadamards, no sign vectors); fp32 accumulation, one
 * rounding to fp16; xh fp16 [rows, k].  Identity rows of xh read W_inner out exactly.  The rows run through the kernel
 * that serves the same row count in a linear: below 65 rows the decode-GEMV (one 16-row group per launch, two decoded
 * tiles per MFMA), from 65 rows the prefill decode-GEMM.  Replaces exl3_gemm_marlin (cuda/csrc/exl3_marlin.cu:411-423),
 * the one-hot test entry of cuda/src/sglang_exl3/parity/marlin_parity.py:149-159. */
int exl3_gemm_rotated(const void* xh, int rows, int k, const void* trellis, int n, int K, int codebook, void* out,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free form of exl3_linear.  No counterpart in the reference: it is for callers that cannot allocate or
 * pass device memory of their own (code under HIP-graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments as exl3_linear without the workspace, and the same results up to 16 rows (past 16 rows
 * it runs one launch per 16 rows, where exl3_linear shares each decoded tile among up to 64 rows: the two then agree
 * to rounding): the split counters and fp32 partials live in a scratch array of EXL3_NOALLOC_SCRATCH_BYTES that the
 * library holds on every GPU it runs on until the process ends, on the GPU of `stream` (the current device for the
 * null stream).  It calls no allocating routine.  A call whose
 * workspace need (that of 16-row launches; exl3_linear_workspace_bytes up to 16 rows) exceeds the scratch returns
 * EXL3_ERR_INVALID and launches nothing.  All calls on one GPU share its scratch: calls that overlap
 * in time on one GPU (several streams, several host threads without ordering) race and give wrong results; calls
 * ordered on one stream are safe, and each leaves the counters at zero for the next. */
#define EXL3_NOALLOC_SCRATCH_BYTES (32u << 20)
size_t exl3_linear_noalloc_max_bytes(void);
int exl3_linear_noalloc(const void* x, int x_bf16, int rows, int k, const exl3_shard* shards_host, int nshards, int K,
                        int codebook, void* y, int y_bf16, void* stream);

/* ---- prefill decode-GEMM (subsystem 3) ------------------------------------------------------------------------ */
/* Workspace bytes of exl3_linear_prefill for `rows` rows of a group with input width k, n_total output columns and
 * nshards shards: EXL3_WORKSPACE_COUNTER_BYTES of split counters (zero before the first use; every call leaves them
 * zero), the per-shard rotated activations (fp16 [nshards][rows][k]), then fp32 partials of the k-split tail tiles.
 * Depends on the current device's CU count. */
size_t exl3_prefill_workspace_bytes(int rows, int k, int n_total, int nshards);
/* Same contract as exl3_linear for many rows: the input rotation of every shard goes to the workspace, then one
 * fused decode-GEMM launch (weights decoded into LDS, fp16 MFMA, fp32 accumulation, output rotation in the epilogue)
 * writes y.  Tiles that do not fill a whole round of the machine are split along k and summed in a fixed order, so
 * results do not depend on scheduling.  Replaces the reference's prefill branch -- rotation, ExLlamaV3 reconstruct, cuBLAS, rotation
 * (cuda/src/sglang_exl3/runtime/ops.py:36-59, 87-95). */
int exl3_linear_prefill(const void* x, int x_bf16, int rows, int k, const exl3_shard* shards_host, int nshards, int K,
                        int codebook, void* y, int y_bf16, void* workspace, size_t workspace_bytes, void* stream);

/* ---- MoE grouped experts (subsystem 5a) --------------------------------------------------------------------------- */
/* Stacked expert weights of one MoE layer (SiLU-gated, no routed scaling: the contract of the reference's
 * Exl3MoEMethod, cuda/src/sglang_exl3/sglang_glue/moe.py:109-119).  All experts share the codebook; gate and up share
 * one bitrate K_gate_up, down has its own K_down (the reference checks only gate K == up K, moe.py:148-152, and runs
 * the two bitrates separately, cuda/src/sglang_exl3/kernels/reference.py:123-149). */
typedef struct exl3_moe_weights {
  const void* gate_trellis; /* int16 [E][H/16][I/16][16K] */
  const void* up_trellis;   /* int16 [E][H/16][I/16][16K] */
  const void* down_trellis; /* int16 [E][I/16][H/16][16K] */
  const void* gate_suh;     /* fp16 [E][H] */
  const void* gate_svh;     /* fp16 [E][I] */
  const void* up_suh;       /* fp16 [E][H] */
  const void* up_svh;       /* fp16 [E][I] */
  const void* down_suh;     /* fp16 [E][I] */
  const void* down_svh;     /* fp16 [E][H] */
} exl3_moe_weights;

/* Workspace bytes of exl3_moe_forward (split counters, routing lists, fp16 rotated inputs, g|u and down rows, fp32
 * partials).  The
 * counter region (EXL3_WORKSPACE_COUNTER_BYTES, holding num_experts * (2 inter + hidden) / 128 counters) must be
 * zero before the first use; every call leaves it zero. */
size_t exl3_moe_workspace_bytes(int tokens, int top_k, int num_experts, int hidden, int inter, int K_gate_up,
                                int K_down);
/* y[t] = sum_j w[t, j] * down_e(fp16(silu(gate_e(x[t])) * up_e(x[t]))), e = topk_ids[t, j]; every linear is an EXL3
 * linear with its own suh / svh; fp32 combine in slot order; ids outside [0, E) are skipped.  x fp16|bf16 [T, H],
 * topk_ids int32 [T, top_k] (top_k <= 64), topk_weights fp32 [T, top_k], y fp16|bf16 [T, H].  Replaces the five
 * launches of cuda/src/sglang_exl3/kernels/marlin_moe.py:272-294 (moe_had_in, moe_gemm, moe_glu_had_in, moe_gemm,
 * moe_combine; cuda/csrc/exl3_marlin_moe.cu:376-499) and the align step (exl3_marlin_moe.cu:532-594) with four
 * launches (three for a single token).  Calls that share a workspace must not overlap. */
int exl3_moe_forward(const void* x, int x_bf16, int tokens, int hidden, const void* topk_ids, const void* topk_weights,
                     int top_k, int num_experts, int inter, const exl3_moe_weights* weights_host, int K_gate_up,
                     int K_down, int codebook, void* y, int y_bf16, void* workspace, size_t workspace_bytes,
                     void* stream);

/* One K class of a mixed-K MoE layer: the stacked weights of its experts in LOCAL order ([E_c][...] per tensor, as
 * exl3_moe_weights), its bitrates, and its expert map (device int32 [num_experts]: global id -> local id, -1 for
 * experts of other classes).  Replaces the per-class ExpertPack of the reference's MixedPack
 * (cuda/src/sglang_exl3/kernels/marlin_moe.py:135-170). */
typedef struct exl3_moe_class {
  exl3_moe_weights weights;
  const int* expert_map;
  int num_local; /* E_c */
  int K_gate_up, K_down;
} exl3_moe_class;

/* Workspace bytes of exl3_moe_forward_classes (the same layout as exl3_moe_forward's, with one k-split plan shared
 * by the classes).  classes_host holds nclasses entries (only their bitrates are read). */
size_t exl3_moe_classes_workspace_bytes(int tokens, int top_k, int num_experts, int hidden, int inter, int nclasses,
                                        const exl3_moe_class* classes_host);
/* exl3_moe_forward for a layer whose experts come in up to EXL3_MOE_MAX_CLASSES K classes; every expert id in
 * [0, num_experts) must belong to exactly one class.  One routing for the layer, then each class's gate/up and down
 * launches over its own experts (weights at their local ids), one combine.  The same results as exl3_moe_forward on
 * a single class.  Replaces run_mixed (cuda/src/sglang_exl3/kernels/marlin_moe.py:247-272). */
int exl3_moe_forward_classes(const void* x, int x_bf16, int tokens, int hidden, const void* topk_ids,
                             const void* topk_weights, int top_k, int num_experts, int inter,
                             const exl3_moe_class* classes_host, int nclasses, int codebook, void* y, int y_bf16,
                             void* workspace, size_t workspace_bytes, void* stream);

/* ---- MoE per-launch stages (the reference's moe_align_decode, moe_had_in, moe_gemm, moe_glu_had_in, moe_combine:
 * cuda/csrc/exl3_marlin_moe.cu:376-618; run order cuda/src/sglang_exl3/kernels/marlin_moe.py:272-294).  The same
 * arithmetic as exl3_moe_forward, one launch per stage, for callers that drive the stages themselves.  Weights are the
 * stored trellis stacks ([E][k/16][n/16][16K] per projection), not a repacked stack. */

/* Routing in the layout of vLLM's moe_align_block_size for one block size (1..64): the slots of every expert (ids
 * outside [0, num_experts), or mapped to -1 by expert_map, dropped) in ascending expert order, each expert's run
 * padded to a multiple of `block` with the sentinel `slots`; expert_ids[i] = the expert of block i (expert_map[e]
 * when a map is given, else e), -1 past the end; *num_post_padded = the padded length.  Slots keep no particular
 * order inside a run.  sorted_ids holds cap >= slots + num_experts * (block - 1) entries (the sentinel past the
 * end), expert_ids max_blocks >= cap / block.  One workgroup; num_experts <= 1024. */
int exl3_moe_align(const int* topk_ids, int slots, int num_experts, const int* expert_map, int block, int* sorted_ids,
                   int cap, int* expert_ids, int max_blocks, int* num_post_padded, void* stream);

/* Mixed-K layers (e.g. 96 experts at K = 3 and 32 at K = 4): the routing of every class in ONE launch, for up to
 * EXL3_MOE_MAX_CLASSES classes.  Class c gets the layout exl3_moe_align gives with expert_maps_host[c] (device int32
 * [num_experts]: global id -> local id in the class, -1 for experts of other classes) and block size blocks_host[c],
 * into sorted_ids_host[c] (caps_host[c] entries), expert_ids_host[c] (max_blocks_host[c] blocks, local ids) and
 * *num_post_padded_host[c].  Every slot lands in the class its expert belongs to.  The *_host arrays hold nclasses
 * entries each; the pointers in them are device memory.  Replaces moe_align_decode with two classes
 * (cuda/csrc/exl3_marlin_moe.cu:532-618; caller cuda/src/sglang_exl3/kernels/marlin_moe.py:195-221). */
#define EXL3_MOE_MAX_CLASSES 2
int exl3_moe_align_classes(const int* topk_ids, int slots, int num_experts, int nclasses,
                           const int* const* expert_maps_host, const int* blocks_host, int* const* sorted_ids_host,
                           const int* caps_host, int* const* expert_ids_host, const int* max_blocks_host,
                           int* const* num_post_padded_host, void* stream);

/* xh[s * slots + slot][k] = fp16(Had(fp16(x[slot / top_k]) * suh_s[e])) (x fp16 or bf16 [tokens][k]) for every slot
 * with a valid expert e = topk_ids[slot] and every shard s < shards (1 or 2; suh: shards pointers to [E][k] fp16);
 * rows of other slots are not written. */
int exl3_moe_had_in(const void* x, int x_bf16, int tokens, int k, const int* topk_ids, int top_k, int num_experts,
                    const void* const* suh, int shards, void* xh, void* stream);

/* Workspace bytes of exl3_moe_gemm: the counter region (EXL3_WORKSPACE_COUNTER_BYTES, zero before the first use;
 * every call leaves it zero) and fp32 split partials.  0 for bad shapes. */
size_t exl3_moe_gemm_workspace_bytes(int rows, int k, int n, int shards, int max_blocks);

/* The grouped expert GEMM: for every block i < *num_post_padded / block with expert e = expert_ids[i] in
 * [0, num_experts) and every row r = sorted_ids[i * block + j] < rows,
 *   c[r][s * n + col] = fp16(sum_k a[s * rows + r][k] * W_s[e][k][col])          (svh == NULL)
 *   c[r][s * n + ...] = fp16(Had(fp16(acc)) * svh_s[e]) per 128 columns          (svh given: the output transform)
 * for each shard s < shards (1 or 2: gate | up side by side).  a: fp16 [shards * rows][k]; trellis / svh: shards
 * pointers to [E][k/16][n/16][16K] int16 / [E][n] fp16; c: fp16 [rows][shards * n]; other rows of c untouched. */
int exl3_moe_gemm(const void* a, int rows, int k, const void* const* trellis, const void* const* svh, int shards, int n,
                  const int* sorted_ids, const int* expert_ids, const int* num_post_padded, int max_blocks, int block,
                  int num_experts, int K, int codebook, void* c, void* workspace, size_t workspace_bytes,
                  void* stream);

/* For every slot with a valid expert e = topk_ids[slot]: act[slot] = fp16(silu(g) * u) (fp32 SiLU; act may be
 * NULL) and xd[slot] = fp16(Had(fp16(act * suh_down[e]))), from gu fp16 [slots][2 inter] = gate | up. */
int exl3_moe_glu_had_in(const void* gu, int slots, int inter, const int* topk_ids, int num_experts,
                        const void* suh_down, void* act, void* xd, void* stream);

/* y[t] = sum over j of topk_weights[t][j] * yd[t * top_k + j] in fp32, slot order, one rounding (fp16 or bf16 y);
 * slots whose id is outside [0, num_experts) are skipped. */
int exl3_moe_combine(const void* yd, const float* topk_weights, const int* topk_ids, int tokens, int top_k, int hidden,
                     int num_experts, void* y, int y_bf16, void* stream);

/* ---- Quantized-KV paged decode attention (subsystem 5b) ------------------------------------------------------------ */
/* The reference has no quantized-KV decode kernel: its nearest relative is the paged fp8 gather + dequant + blockwise
 * fp16 attention with log-sum-exp merge of xpu/exl3xpu/fp8kv_prefill.py:73-117 (gather_dequant, prefill_attention).
 * Cache (this library's layout): k_cache / v_cache int8 codes [num_pages][Hkv][16][128] (bits = 8) or packed uint8
 * [num_pages][Hkv][16][64] (bits = 4: element 2i in the low nibble, 2i+1 in the high nibble, two's complement);
 * k_scale / v_scale fp16 [num_pages][Hkv]; value = code * scale. */

/* Workspace bytes of exl3_kv_decode_attention (fp32 partial (m, l, O) per chunk of pages).  No zero-fill needed.
 * Not monotone in batch (a smaller batch can take more chunks per sequence); never larger for fewer pages. */
size_t exl3_kv_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int max_pages);
/* out[b][h] = softmax(sm_scale * q[b][h] . K_b^T) V_b over the first seq_lens[b] tokens of sequence b, whose pages are
 * page_table[b][0 .. ceil(seq_lens[b] / 16)); query head h reads KV head h / (Hq / Hkv) (Hq / Hkv <= 16).
 * q fp16 [B][Hq][128], page_table int32 [B][max_pages], seq_lens int32 [B], out fp16 [B][Hq][128].  A sequence of
 * length 0 gives zeros; page ids outside [0, num_pages) are clamped (never read outside the cache).  head_dim must be
 * 128 and page_size 16.  Two launches (split-KV over page chunks, then the log-sum-exp merge), one when a single chunk
 * covers every sequence; deterministic. */
int exl3_kv_decode_attention(const void* q, const void* k_cache, const void* v_cache, const void* k_scale,
                             const void* v_scale, int num_pages, const void* page_table, int max_pages,
                             const void* seq_lens, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                             int page_size, int bits, float sm_scale, void* out, void* workspace,
                             size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_MI355X_H */
