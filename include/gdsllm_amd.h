/*
 * gdsllm_amd — C ABI of the MI355X (gfx950) quantized-weight matvec library.
 *
 * Every entry point takes raw device pointers, 64-bit sizes and a HIP stream
 * (passed as `void*`, 0 = the null stream), enqueues its kernels asynchronously
 * on that stream and returns a status code.  A non-zero status leaves a
 * human-readable message in gdsllm_last_error() (thread-local).  Argument
 * validation happens before any HIP call, so a rejected call never touches
 * the device.
 *
 * Weight formats (byte layouts are the ones the reference's converters write
 * and its kernels read):
 *   Q4_0   row-major [rows][cols/32] blocks of 18 bytes: fp16 d (LE) + 16 bytes
 *          qs; element 32b+j = d*((qs[j]&15)-8), element 32b+j+16 = d*((qs[j]>>4)-8)
 *          (runtime/gguf_dequant.cu:84-107, runtime/fused_gemv.cu:63-71)
 *   Q8_0   row-major blocks of 34 bytes: fp16 d + int8 qs[32]; element = d*qs[i]
 *          (runtime/gguf_dequant.cu:40-57)
 *   affine uint32 words [rows][cols/8], 8 nibbles LSB-first, fp16 scale and bias
 *          per group of `group_size` consecutive elements of a row;
 *          element = nib*scale + bias (runtime/affine_q4_dequant.cu:28-59)
 * Activations and outputs are fp16; every reduction accumulates in fp32.
 */
#ifndef GDSLLM_AMD_H
#define GDSLLM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum gdsllm_status {
    GDSLLM_OK = 0,
    GDSLLM_ERR_INVALID_ARGUMENT = 1, /* shape / size / pointer rejected          */
    GDSLLM_ERR_UNSUPPORTED = 2,      /* valid request this build cannot serve    */
    GDSLLM_ERR_HIP = 3,              /* a HIP runtime call or launch failed      */
    GDSLLM_ERR_IO = 4,               /* file open / read failed                  */
    GDSLLM_ERR_OUT_OF_MEMORY = 5     /* device allocation failed                 */
};

/* Message of the last failing call on this host thread ("" if none). */
const char* gdsllm_last_error(void);
/* Library version string. */
const char* gdsllm_version(void);

/* ---------------------------------------------------------------- buffers --
 * HBM-resident weight buffers.  Replace the cuFile buffer lifecycle
 * gds_alloc / gds_free / gds_read (runtime/gds_io.cu:93-118, 120-131,
 * 135-191) behind the same GdsBufferHandle shape (runtime/gds_bindings.cpp:51-76):
 * sizes round up to 4 KiB like gds_alloc (runtime/gds_io.cu:97-99), reads are
 * pread() into pinned host staging followed by hipMemcpy into the buffer.  */
int gdsllm_buffer_alloc(size_t size, int device_id, void** dev_ptr, size_t* rounded_size);
int gdsllm_buffer_free(void* dev_ptr, int device_id);
/* Read `size` bytes of `path` starting at `file_offset` into dev_ptr+buf_offset.
 * `buf_size` is the buffer's size, checked like gds_read (runtime/gds_io.cu:140-142).
 * *bytes_read receives the count copied (short only at end of file).
 * Blocking: returns once the bytes are in HBM.  Four reader threads share the
 * work in 8 MiB chunks through a per-device pinned staging pool (64 MiB, kept
 * until the process ends); reads on one device run one at a time.         */
int gdsllm_buffer_read_file(void* dev_ptr, size_t buf_size, const char* path,
                            size_t size, int64_t file_offset, int64_t buf_offset,
                            int device_id, int64_t* bytes_read);

/* ---------------------------------------------------------------- dequant --
 * Bit-exact fp16 dequantization: every element is one IEEE round-to-nearest-even
 * of the exact fp32 value the reference computes.                            */

/* Replaces launch_dequant_q4_0 (runtime/gguf_dequant.h:25-26,
 * runtime/gguf_dequant.cu:110-118).  dst: fp16[num_blocks*32].            */
int gdsllm_dequant_q4_0(const void* src, void* dst, int64_t num_blocks, void* stream);
/* Replaces launch_dequant_q8_0 (runtime/gguf_dequant.h:19-20,
 * runtime/gguf_dequant.cu:60-68).  dst: fp16[num_blocks*32].              */
int gdsllm_dequant_q8_0(const void* src, void* dst, int64_t num_blocks, void* stream);
/* Embedding lookup over a GGUF table [vocab][hidden]: out[t] = the fp16
 * dequantized row token_ids[t] (bit-exact as above), zeros for an id outside
 * [0, vocab).  Replaces the reference's dequantize-the-whole-table-then-
 * F.embedding (runtime/scheduler.py:22-35) by a gather of the needed rows.
 * hidden % 64 == 0; token_ids: int64 on device; out: fp16[n_tokens][hidden].
 * At most 65535 tokens per call.                                             */
int gdsllm_embed_q4_0(const void* table, const int64_t* token_ids, int64_t n_tokens,
                      int64_t vocab, int64_t hidden, void* out, void* stream);
int gdsllm_embed_q8_0(const void* table, const int64_t* token_ids, int64_t n_tokens,
                      int64_t vocab, int64_t hidden, void* out, void* stream);
/* Replaces launch_dequant_affine_q4 (runtime/affine_q4_dequant.h:29-32,
 * runtime/affine_q4_dequant.cu:61-73).  Elements are grouped by flat index
 * (group = i / group_size) exactly as the reference does; `in_dim` is checked
 * to be a multiple of group_size and otherwise unused, as in the reference.  */
int gdsllm_dequant_affine_q4(const void* weight, const void* scales, const void* biases,
                             void* dst, int64_t num_elements, int64_t in_dim,
                             int64_t group_size, void* stream);

/* ------------------------------------------------------------ fused GEMV --
 * y[b][r] = fp16( sum_k W[r][k] * x[b][k] ), b < batch (1..8), fp32 accumulate.
 * x row b starts at x + b*ldx elements, y row b at y + b*ldy elements.
 * out_dim == 0 or in_dim == 0 is a no-op, as in the reference launchers.      */

/* Replaces launch_fused_q4_0_gemv (runtime/fused_gemv.h:23-25,
 * runtime/fused_gemv.cu:107-135); batch > 1 is an extension.                 */
int gdsllm_fused_q4_0_gemv(const void* weight, const void* x, void* y,
                           int64_t out_dim, int64_t in_dim, int64_t batch,
                           int64_t ldx, int64_t ldy, void* stream);
/* Replaces launch_fused_q8_0_gemv (runtime/fused_gemv.h:29-31,
 * runtime/fused_gemv.cu:207-231).                                            */
int gdsllm_fused_q8_0_gemv(const void* weight, const void* x, void* y,
                           int64_t out_dim, int64_t in_dim, int64_t batch,
                           int64_t ldx, int64_t ldy, void* stream);
/* ------------------------------------------------- per-column int8 weights --
 * The converter's "int8" format (tools/convert_weights.py:55-83): W int8
 * [out_dim][in_dim] row-major, scale fp16 [in_dim] (one per input column).
 * Replace the projection runtime/llama.py:162-165 computes from it,
 * w = (w.float() * scale).half(); F.linear(x, w), which dequantizes the whole
 * matrix through fp32 on every call.                                         */

/* dst fp16[rows][cols] = RN16(w * scale[col]): bit-exact with the reference's
 * (w.float() * scale).half().                                                */
int gdsllm_dequant_int8(const void* weight, const void* scale, void* dst, int64_t rows, int64_t cols,
                        void* stream);
/* y[b][r] = sum_k RN16(w[r][k] * scale[k]) * x[b][k] with fp32 accumulation,
 * batch 1..8, x rows ldx apart, y rows ldy apart.  The fast path needs
 * in_dim % 16 == 0, 16-byte aligned weight, scale and x (ldx % 8 == 0 when
 * batch > 1); other shapes run a slower kernel with the same results.        */
int gdsllm_fused_int8_gemv(const void* weight, const void* scale, const void* x, void* y, int64_t out_dim,
                           int64_t in_dim, int64_t batch, int64_t ldx, int64_t ldy, void* stream);

/* ----------------------------------------------------- decode-step fusions --
 * No counterpart in the reference, which issues one dequant_linear per
 * projection: q/k/v of one layer read the same x (runtime/llama.py:212-214),
 * and the MLP computes F.silu(gate) * up before the down projection
 * (runtime/llama.py:253-256).  For decode loops that want fewer launches.     */

/* n (1..4) GEMVs sharing x and in_dim in one launch: ys[i] receives
 * fp16[batch][out_dims[i]] (row-contiguous) = W_i x.  Same numerics as
 * gdsllm_fused_q4_0_gemv / gdsllm_fused_q8_0_gemv on each matrix (the same
 * bits, except where the single GEMV of a matrix too short to give every
 * compute unit a workgroup, with in_dim over 2-4 windows of 4096, adds its
 * window sums in another order, and for Q4_0 at batch 3-8, where the group
 * launch sums the same block products in the x-in-registers kernel's order:
 * equal to fp32 rounding); shapes no single-launch kernel serves (batch 3-8
 * Q8_0, in_dim > 8192 or not a multiple of 256 at batch 3-8, unaligned
 * weights or x) fall back to one launch per matrix.                          */
int gdsllm_fused_q4_0_gemv_group(int n, const void* const* weights, void* const* ys,
                                 const int64_t* out_dims, const void* x, int64_t in_dim,
                                 int64_t batch, int64_t ldx, void* stream);
int gdsllm_fused_q8_0_gemv_group(int n, const void* const* weights, void* const* ys,
                                 const int64_t* out_dims, const void* x, int64_t in_dim,
                                 int64_t batch, int64_t ldx, void* stream);
/* h[b][r] = fp16(silu(g) * u) with g = fp16((W_gate x_b)[r]), u = fp16((W_up x_b)[r])
 * and torch's fp16 semantics (silu in fp32 rounded to fp16, then the product
 * rounded to fp16), in one launch; gate and up outputs never reach memory.
 * Needs in_dim % 256 == 0, 16-byte aligned weights and x with ldx % 8 == 0,
 * and at batch 3-8 Q4_0 with in_dim <= 8192 (else GDSLLM_ERR_UNSUPPORTED).  */
int gdsllm_fused_q4_0_gate_up_silu(const void* w_gate, const void* w_up, const void* x, void* h,
                                   int64_t out_dim, int64_t in_dim, int64_t batch, int64_t ldx,
                                   int64_t ldh, void* stream);
int gdsllm_fused_q8_0_gate_up_silu(const void* w_gate, const void* w_up, const void* x, void* h,
                                   int64_t out_dim, int64_t in_dim, int64_t batch, int64_t ldx,
                                   int64_t ldh, void* stream);

/* Replaces launch_fused_affine_q4_gemv (runtime/affine_q4_dequant.h:41-44,
 * runtime/affine_q4_dequant.cu:160-187).                                     */
int gdsllm_fused_affine_q4_gemv(const void* weight, const void* scales, const void* biases,
                                const void* x, void* y, int64_t out_dim, int64_t in_dim,
                                int64_t group_size, int64_t batch, int64_t ldx,
                                int64_t ldy, void* stream);

/* ------------------------------------------------------ MoE expert gather --
 * One projection of a stacked affine-Q4 expert tensor as the Qwen-MoE layer
 * file stores it: words [E][out_dim][in_dim/8], then scales and biases
 * [E][out_dim][in_dim/group_size], each region at its own offset
 * (tools/convert_qwen_moe.py:216-233).  Expert e's slices start at
 * weight + e*weight_stride, scales + e*scale_stride, biases + e*bias_stride
 * (bytes; runtime/torch_bridge.py:326-337).                                   */
typedef struct gdsllm_affine_experts {
    const void* weight;
    const void* scales;
    const void* biases;
    int64_t weight_stride;
    int64_t scale_stride;
    int64_t bias_stride;
    int64_t num_experts;
    int64_t out_dim;
    int64_t in_dim;
    int64_t group_size;
} gdsllm_affine_experts;

/* Bytes of device workspace gdsllm_moe_gather_affine_q4 needs. */
size_t gdsllm_moe_gather_workspace_size(int64_t top_k, int64_t ffn_dim);

/* Top-k expert-gather MLP for one token (decode):
 *   y = fp16( sum_k w[k] * down[idx[k]] . h_k ),
 *   h_k = fp16( fp16(silu(fp16(gate[idx[k]] . x))) * fp16(up[idx[k]] . x) )
 * i.e. the decode branch of moe_mlp_selective (runtime/qwen_moe.py:455-474)
 * with the routing weights combined in fp32.  idx: int32[top_k] on device,
 * routing_weights: fp16[top_k] on device, x: fp16[hidden], y: fp16[hidden].
 * gate/up: out_dim = ffn_dim, in_dim = hidden; down: out_dim = hidden,
 * in_dim = ffn_dim.  Expert indices outside [0, num_experts) contribute
 * nothing.  No counterpart kernel exists in the reference, which loops over
 * fused_affine_q4_gemv launches in Python.                                   */
int gdsllm_moe_gather_affine_q4(const gdsllm_affine_experts* gate,
                                const gdsllm_affine_experts* up,
                                const gdsllm_affine_experts* down,
                                const void* x, const int32_t* idx,
                                const void* routing_weights, int64_t top_k,
                                void* y, void* workspace, size_t workspace_bytes,
                                void* stream);
/* The same gather with no workspace argument and no allocation of any kind:
 * its gate/up/h workspace is a fixed device array of
 * gdsllm_moe_gather_noalloc_max_bytes() bytes (1 MiB) inside the library, one
 * per device, held until the process ends.  No counterpart in the reference;
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Rejects
 * top_k * ffn_dim whose workspace (gdsllm_moe_gather_workspace_size) exceeds
 * that size.  Calls that overlap on one device share the array and race: the
 * caller orders them (one stream, or events between streams).               */
size_t gdsllm_moe_gather_noalloc_max_bytes(void);
int gdsllm_moe_gather_affine_q4_noalloc(const gdsllm_affine_experts* gate,
                                        const gdsllm_affine_experts* up,
                                        const gdsllm_affine_experts* down,
                                        const void* x, const int32_t* idx,
                                        const void* routing_weights, int64_t top_k,
                                        void* y, void* stream);
/* The whole decode MoE MLP of qwen_moe.py:455-513 after routing, in two
 * launches: the top_k routed experts and the shared expert (one-expert
 * descriptors shared_gate/shared_up [1][F][H], shared_down [1][H][F]) share
 * the gate/up launch, which also computes the shared-expert gate logit
 * g = fp16(shared_gate_weight . x) (fp16 [H], the bits gdsllm_gemv_f16 gives);
 * the down launch applies the shared expert and the combine:
 * y = clamp(fp16(sum_k w_k * down_k(h_k)) +
 * fp16(fp16(sigmoid(g)) * fp16(shared_down(h_s))), +-65504), the rounding of
 * gdsllm_moe_combine.  No counterpart in the reference, which issues ~40
 * launches for it.  Needs the row-span shapes of gdsllm_moe_gather_affine_q4
 * with top_k + 1 slots, a shared expert of the routed width and grouping, and
 * x and shared_gate_weight on the 16-byte grid (else GDSLLM_ERR_UNSUPPORTED);
 * workspace_bytes >= gdsllm_moe_step_workspace_size(top_k, F).              */
size_t gdsllm_moe_step_workspace_size(int64_t top_k, int64_t ffn_dim);
int gdsllm_moe_step_affine_q4(const gdsllm_affine_experts* gate, const gdsllm_affine_experts* up,
                              const gdsllm_affine_experts* down, const gdsllm_affine_experts* shared_gate,
                              const gdsllm_affine_experts* shared_up, const gdsllm_affine_experts* shared_down,
                              const void* x, const int32_t* idx, const void* routing_weights, int64_t top_k,
                              const void* shared_gate_weight, void* y, void* workspace, size_t workspace_bytes,
                              void* stream);
/* The same step with the routing of qwen_moe.py:386-416 folded in, in three
 * launches: the fp16 router GEMV (gdsllm_gemv_f16 on router_weight
 * [num_experts][H], logits into the workspace), then the gate/up launch, each
 * of whose waves takes the top_k picks of those logits itself (the selection
 * and fp16 softmax of gdsllm_moe_route_topk, bit for bit), then the down launch.
 * idx_out (int32 [top_k]) and weights_out (fp16 [top_k]) receive the picks in
 * descending order and their weights, as moe_route returns them.  No
 * counterpart in the reference (moe_route followed by moe_mlp_selective).
 * num_experts = gate->num_experts <= 512 and a multiple of 8, router_weight
 * and x on the 16-byte grid (else GDSLLM_ERR_UNSUPPORTED or
 * GDSLLM_ERR_INVALID_ARGUMENT); workspace_bytes >=
 * gdsllm_moe_step_routed_workspace_size(top_k, F, num_experts).             */
size_t gdsllm_moe_step_routed_workspace_size(int64_t top_k, int64_t ffn_dim, int64_t num_experts);
int gdsllm_moe_step_routed_affine_q4(const void* router_weight, const gdsllm_affine_experts* gate,
                                     const gdsllm_affine_experts* up, const gdsllm_affine_experts* down,
                                     const gdsllm_affine_experts* shared_gate, const gdsllm_affine_experts* shared_up,
                                     const gdsllm_affine_experts* shared_down, const void* x, int64_t top_k,
                                     const void* shared_gate_weight, void* y, int32_t* idx_out, void* weights_out,
                                     void* workspace, size_t workspace_bytes, void* stream);

/* --------------------------------------- on-device MoE routing, epilogue --
 * The reference routes on the host side of a sync (F.linear, torch.topk,
 * softmax, .tolist(); runtime/qwen_moe.py:386-416) and finishes the MoE MLP
 * with elementwise torch ops (runtime/qwen_moe.py:496-513).  These keep the
 * whole step on the device, feeding gdsllm_moe_gather_affine_q4 directly.   */

/* y[b][r] = fp16( sum_k w[r][k] * x[b][k] ), fp16 weights row-major
 * [out_dim][in_dim], fp32 accumulation, batch <= 8.  Replaces F.linear on the
 * fp16 router (runtime/qwen_moe.py:408) and on the shared-expert gate
 * (runtime/qwen_moe.py:505-508).                                            */
int gdsllm_gemv_f16(const void* weight, const void* x, void* y,
                    int64_t out_dim, int64_t in_dim, int64_t batch,
                    int64_t ldx, int64_t ldy, void* stream);

/* Per token t < n_tok, from fp16 logits at logits + t*ld_logits: the top_k
 * largest in descending order into idx[t*top_k ...] (int32) and
 * fp16(softmax_fp32(picked logits)) into weights[t*top_k ...].  Ties go to
 * the lower expert index, NaN ranks above every number, -0 equals +0.
 * num_experts <= 4096, top_k <= min(64, num_experts).  Replaces torch.topk +
 * F.softmax(.float()).type_as(x) (runtime/qwen_moe.py:410-412).              */
int gdsllm_moe_route_topk(const void* logits, int64_t num_experts,
                          int64_t n_tok, int64_t ld_logits, int64_t top_k,
                          int32_t* idx, void* weights, void* stream);

/* y = clamp(expert_out + fp16(fp16(sigmoid(g_t)) * shared_out), +-65504)
 * elementwise over n_tok rows of `hidden` fp16 values, g_t = the fp16 shared-
 * expert gate logit of token t (shared_gate_logit[t]); each op in fp32 rounded
 * to fp16 as torch does on fp16 tensors, NaN kept.  Replaces
 * runtime/qwen_moe.py:508-513.                                              */
int gdsllm_moe_combine(const void* expert_out, const void* shared_out,
                       const void* shared_gate_logit, void* y,
                       int64_t hidden, int64_t n_tok, void* stream);

/* ---------------------------------------------------- prefill dequant-GEMM --
 * Y[t][r] = fp16( sum_k X[t][k] * W[r][k] ), t < tokens, on MFMA.  Replaces
 * the prefill branch dequant -> F.linear (runtime/llama.py:160-166).
 * X row t at x + t*ldx, Y row t at y + t*ldy (elements).                     */
int gdsllm_dequant_gemm_q4_0(const void* weight, const void* x, void* y,
                             int64_t out_dim, int64_t in_dim, int64_t tokens,
                             int64_t ldx, int64_t ldy, void* stream);

/* The same on Q8_0 weights.  Replaces dequant_gguf(..., "q8_0") -> F.linear
 * (runtime/llama.py:160-166).  Needs in_dim % 256 == 0, 16-byte aligned
 * weight and x rows (else GDSLLM_ERR_UNSUPPORTED: the caller keeps the
 * dequant route).  W enters the matrix cores as the bit-exact dequantized
 * fp16 value (runtime/gguf_dequant.cu:52-57).                               */
int gdsllm_dequant_gemm_q8_0(const void* weight, const void* x, void* y,
                             int64_t out_dim, int64_t in_dim, int64_t tokens,
                             int64_t ldx, int64_t ldy, void* stream);

/* The same on affine-Q4 weights (words [out_dim][in_dim/8], scales and biases
 * [out_dim][in_dim/group_size]).  Replaces _dequant_affine_q4 -> F.linear
 * (runtime/qwen_moe.py:69-73).  Needs in_dim % 256 == 0, group_size 32, 64
 * or 128, 16-byte aligned words and x rows, scales/biases 4-byte aligned
 * (16-byte for group_size 32), else GDSLLM_ERR_UNSUPPORTED.  Each weight is
 * fp16(nib*scale + bias) rounded once; the reference rounds through fp32
 * first (runtime/affine_q4_dequant.cu:50-58), which differs by one fp16 ulp
 * of a weight only where nib*scale + bias is not exact in fp32.            */
int gdsllm_dequant_gemm_affine_q4(const void* weight, const void* scales, const void* biases,
                                  const void* x, void* y, int64_t out_dim, int64_t in_dim,
                                  int64_t group_size, int64_t tokens, int64_t ldx, int64_t ldy,
                                  void* stream);
/* The MLP input of a prefill chunk in one launch: h[t][r] =
 * fp16(fp16(silu(g)) * u) with g = fp16(sum_k x[t][k] * gate[r][k]) and u
 * likewise for up (GGUF Q4_0 / Q8_0 [ffn_dim][in_dim]; g and u are the bits
 * gdsllm_dequant_gemm_* gives for each when both take the same row tile,
 * else equal up to fp32 reassociation of each row's sum: 256-row tiles add
 * two K halves, 128-row tiles four K quarters), torch's fp16 SiLU and product.
 * Replaces the reference's two prefill projections and its elementwise SiLU
 * (runtime/llama.py:253-256 over dequant_linear, llama.py:160-166); the
 * prefill form of gdsllm_fused_*_gate_up_silu.  in_dim % 256 == 0, weights
 * and x on the 16-byte grid, ldx % 8 == 0 (else GDSLLM_ERR_UNSUPPORTED).     */
int gdsllm_dequant_gemm_gate_up_silu_q4_0(const void* gate_weight, const void* up_weight, const void* x,
                                          void* h, int64_t ffn_dim, int64_t in_dim, int64_t tokens,
                                          int64_t ldx, int64_t ldh, void* stream);
int gdsllm_dequant_gemm_gate_up_silu_q8_0(const void* gate_weight, const void* up_weight, const void* x,
                                          void* h, int64_t ffn_dim, int64_t in_dim, int64_t tokens,
                                          int64_t ldx, int64_t ldh, void* stream);

/* Bytes of device workspace gdsllm_moe_prefill_affine_q4 needs. */
size_t gdsllm_moe_prefill_workspace_size(int64_t tokens, int64_t top_k, int64_t ffn_dim,
                                         int64_t hidden, int64_t num_experts);

/* Routed-expert MLP of a prefill chunk over stacked affine-Q4 experts
 * (layout of gdsllm_moe_gather_affine_q4): the prefill branch of
 * moe_mlp_selective (runtime/qwen_moe.py:475-492).  idx int32 [tokens][top_k]
 * and routing_weights fp16 [tokens][top_k] on the device, x row t at
 * x + t*ldx, expert_output row t at y + t*ldy (fp16 [hidden]):
 *   y[t] = sum over j in order of fp16(w[t][j] * down_e(h)), each product and
 *          partial sum rounded to fp16, e = idx[t][j],
 *   h    = fp16(fp16(silu(fp16(gate_e . x_t))) * fp16(up_e . x_t)).
 * Four launches and no host sync: the entries sorted by expert, one grouped
 * MFMA GEMM for gate/up/SiLU over each expert's tokens, one for down, the
 * combine.  Expert indices outside [0, num_experts) contribute nothing.  No
 * counterpart kernel in the reference, which loops over the unique experts
 * with dequant -> F.linear per projection.  Needs hidden and ffn multiples of
 * 256, group_size 32, 64 or 128, gate and up with equal strides, at most 4096
 * experts (else GDSLLM_ERR_UNSUPPORTED); workspace_bytes >=
 * gdsllm_moe_prefill_workspace_size(tokens, top_k, ffn, hidden, experts).    */
int gdsllm_moe_prefill_affine_q4(const gdsllm_affine_experts* gate,
                                 const gdsllm_affine_experts* up,
                                 const gdsllm_affine_experts* down,
                                 const void* x, int64_t ldx, const int32_t* idx,
                                 const void* routing_weights, int64_t tokens, int64_t top_k,
                                 void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* ------------------------------------------------------ measurement helpers --
 * Not on the matvec path and with no counterpart in the reference: reference
 * kernels the benchmark measures the GEMV against on the same device.
 * gdsllm_read_stream reads `bytes` at src once (16-byte non-temporal loads,
 * `workgroups` workgroups of 256 threads) and discards the data; sink must
 * hold `workgroups` uint32 (written only when a workgroup's XOR of its data
 * equals `key`).  gdsllm_empty_launch launches a kernel with no work.       */
int gdsllm_read_stream(const void* src, int64_t bytes, int64_t workgroups, uint32_t key, void* sink,
                       void* stream);
int gdsllm_empty_launch(int64_t workgroups, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDSLLM_AMD_H */
