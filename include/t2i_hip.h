/*
 * t2i_hip.h -- C ABI of the MI355X (gfx950) W4A16 hot path.
 *
 * Every pointer is a device pointer unless stated otherwise; `stream` is a
 * hipStream_t (NULL = the legacy default stream).  All calls are
 * stream-ordered and asynchronous; nothing here allocates device memory.
 *
 * Return codes: 0 ok; > 0 a hipError_t from the launch; < 0 an argument
 * error (see T2I_ERR_*), detected on the host before anything is launched.
 * t2i_last_error() gives a thread-local message for the last failure.
 *
 * Weight format: AutoGPTQ group-wise int4, unchanged from the checkpoint:
 *   qweight int32 [K/8, N]   nibble j of word (r, n) = q[8r + j][n]
 *   qzeros  int32 [K/g, N/8] nibble j of word (t, c) = stored zero of column 8c + j;
 *                            effective zero = stored + 1
 *   scales  fp16  [K/g, N]
 * W[n][k] = (q[k][n] - z[k/g][n]) * s[k/g][n].  Group size g = 128.
 * Activations are bf16 (uint16_t bit patterns), row-major, 16-byte aligned.
 *
 * Workspace: the split-context attention keeps per-split partial results and
 * one arrival counter per (sequence, kv head) in a caller-owned workspace sized
 * by t2i_decode_attention_workspace_bytes().  The workspace must be zero-filled
 * before its first use; every call leaves the counters at zero again, so a
 * captured graph can replay the call without a memset.  Calls that overlap in
 * time (different streams) must not share a workspace.
 */
#ifndef T2I_HIP_H
#define T2I_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define T2I_ABI_VERSION 7
#define T2I_MAX_ROWS (65535 * 16)   /* rows of one linear call: 16-row tiles in grid.z */

#define T2I_OK 0
#define T2I_ERR_NULL (-1)      /* a required pointer is NULL */
#define T2I_ERR_SHAPE (-2)     /* a size is not supported (K % 128, N % 16, M range, ...) */
#define T2I_ERR_ALIGN (-3)     /* a pointer is not 16-byte aligned */
#define T2I_ERR_GROUP (-4)     /* group size other than 128 */
#define T2I_ERR_WORKSPACE (-5) /* workspace missing or too small */
#define T2I_ERR_VALUE (-6)     /* a scalar argument is out of range */

int t2i_abi_version(void);
const char* t2i_strerror(int code);
const char* t2i_last_error(void);

/* ---------------------------------------------------------------------------
 * Dequantisation hook (bit-exact check of the unpack and zero convention).
 * W_nk fp32 [N, K] = (q - z) * s, exact in fp32.
 * Replaces: fast_qwen3/fast_packed_format.py:132-161 (_autogptq_linear_to_dense)
 *           and quantized_qwen3/packed_format.py:88-106 (nibble unpack, zero + 1).
 */
int t2i_w4a16_dequant_f32(const int32_t* qweight, const int32_t* qzeros,
                          const uint16_t* scales, int32_t K, int32_t N,
                          int32_t group_size, float* W_nk, void* stream);

/* ---------------------------------------------------------------------------
 * W4A16 linear: y[M, N] = x[M, K] . W^T, fp32 accumulation, bf16 output.
 * 1 <= M <= T2I_MAX_ROWS; K % 128 == 0; N % 16 == 0.  M = 1 is the GEMV case,
 * M up to 64 the batched decode, larger M a prompt (prefill) batch.
 * residual (nullable, may alias y): y = bf16(bf16(x.W^T) + residual).
 * Replaces: quantized_qwen3/operators/w4a16_gemv/op.py:22-126 (W4A16GEMV, M = 1)
 *           quantized_qwen3/operators/w4a16_gemm/op.py:23-174, 267-333
 *           (W4A16GEMM / W4A16KGroupGEMM, M = 4..32 on the NPU)
 *           and the CPU oracle quantized_qwen3/model.py:133-146.
 * Residual form replaces fast_qwen3/operators/q4nx_fused_linear_residual_projection/op.py:31-118.
 */
int t2i_w4a16_linear(const uint16_t* x, int32_t M,
                     const int32_t* qweight, const int32_t* qzeros,
                     const uint16_t* scales, int32_t K, int32_t N, int32_t group_size,
                     const uint16_t* residual, uint16_t* y, void* stream);

/* ---------------------------------------------------------------------------
 * Paired gate/up linear over one weight whose columns alternate gate and up
 * (fused column 2i = gate i, 2i+1 = up i; N = 2*I, N % 32 == 0).  swiglu != 0: h[M, I] = bf16(bf16(silu(bf16 gate)) * bf16 up) into y0,
 * y1 unused.  swiglu == 0: y0 = gate [M, I], y1 = up [M, I].
 * Replaces: quantized_qwen3/operators/w4a16_gemm/op.py:178-263 (W4A16PairedKGroupGEMM,
 *           gate = pair 0, up = pair 1) + torch2iron/operators/silu_mul (SiLUMul).
 */
int t2i_w4a16_gate_up(const uint16_t* x, int32_t M,
                      const int32_t* qweight, const int32_t* qzeros,
                      const uint16_t* scales, int32_t K, int32_t N, int32_t group_size,
                      int32_t swiglu, uint16_t* y0, uint16_t* y1, void* stream);

/* ---------------------------------------------------------------------------
 * RMSNorm fused into the linear: y = inv * W4A16(bf16(x * norm_weight)) per row,
 * inv = bf16(rsqrt(mean(x^2)+eps)) as t2i_rmsnorm rounds it.  This equals
 * W4A16(RMSNorm(x)) up to where the products are rounded to bf16 (the norm scale
 * multiplies the fp32 sums instead of each activation).  Limits as
 * t2i_w4a16_linear / t2i_w4a16_gate_up.  x is the un-normalised residual stream [M, K].
 * Replaces: fast_qwen3/operators/q4nx_fused_qkv_projection/op.py:30-136
 *           (Q4NXFusedQKVProjection: hidden, norm_weight, W, out) and
 *           fast_qwen3/operators/q4nx_fused_up_gate_projection/op.py:30-126
 *           (Q4NXFusedUpGateProjection), with the RMSNorm + projection of
 *           quantized_qwen3/batch_decode_fused.py:426-530.
 */
int t2i_w4a16_rmsnorm_linear(const uint16_t* x, int32_t M, const uint16_t* norm_weight, float eps,
                             const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                             int32_t K, int32_t N, int32_t group_size, uint16_t* y, void* stream);
int t2i_w4a16_rmsnorm_gate_up(const uint16_t* x, int32_t M, const uint16_t* norm_weight, float eps,
                              const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                              int32_t K, int32_t N, int32_t group_size, int32_t swiglu,
                              uint16_t* y0, uint16_t* y1, void* stream);

/* ---------------------------------------------------------------------------
 * Decode-linear weights in tiles.  t2i_w4a16_tile_qweight writes a copy of an
 * AutoGPTQ qweight [K/8, N] into `tiles` (K/8 * N int32, not overlapping it),
 * grouped so that the decode linear reads each workgroup's weights as whole,
 * contiguous lines: one 256-word tile per (16-column block cb, 128-deep group g)
 * at word (cb * K/128 + g) * 256, holding word row 4 j + r of the group, column
 * 16 cb + c at (16 r + c) * 4 + j (j, r < 4; c < 16).  A permutation: no value
 * changes.  Done once per weight (like the reference's repack into its NPU
 * layout, fast_qwen3/fast_packed_format.py:132-161), stream-ordered.
 *
 * t2i_w4a16_linear_tiles is t2i_w4a16_linear / t2i_w4a16_gate_up /
 * t2i_w4a16_rmsnorm_linear / t2i_w4a16_rmsnorm_gate_up over such tiles: same
 * kernels, same arithmetic, bit-identical outputs.  qweight (may be NULL) is the
 * AutoGPTQ original: given, the call also serves prompt rows (M >= 512 without
 * the fused norm, which read qweight) and reads qweight for the few decode plans
 * that read it faster; NULL: every plan reads the tiles, and prompt rows are
 * rejected (T2I_ERR_SHAPE).  epilogue:
 * T2I_TILES_STORE (y0 = y, or y0 = bf16(bf16(y) + residual) with residual != NULL),
 * T2I_TILES_SWIGLU (paired weight, y0 = h) or T2I_TILES_PAIRED (y0 = gate, y1 = up).
 * norm_weight != NULL: the fused RMSNorm (no residual).
 * No counterpart in the reference's call surface beyond the repack it mirrors:
 * for callers that keep decode weights resident (the batch-decode driver).
 */
#define T2I_TILES_STORE 0
#define T2I_TILES_SWIGLU 1
#define T2I_TILES_PAIRED 2
int t2i_w4a16_tile_qweight(const int32_t* qweight, int32_t K, int32_t N, int32_t* tiles, void* stream);
int t2i_w4a16_linear_tiles(const uint16_t* x, int32_t M, const uint16_t* norm_weight, float eps,
                           const int32_t* qweight, const int32_t* tiles, const int32_t* qzeros,
                           const uint16_t* scales, int32_t K, int32_t N, int32_t group_size,
                           int32_t epilogue, const uint16_t* residual, uint16_t* y0, uint16_t* y1,
                           void* stream);

/* ---------------------------------------------------------------------------
 * Chained RMSNorm between decode linears over tiles (the decode layer's
 * o_proj -> RMSNorm -> gate_up and down -> RMSNorm -> next qkv): the producer
 * writes the next norm's input, the consumer takes it pre-multiplied.
 *   producer: next_norm_weight, xg_out, sumsq_out given, residual epilogue
 *     (T2I_TILES_STORE with residual): y0 as t2i_w4a16_linear_tiles, and also
 *     xg_out[m][n] = bf16(y0[m][n] * next_norm_weight[n]) and sumsq_out[m][b] =
 *     sum over the 16 columns of block b of y0[m][n]^2 (fp32, [M][N/16]).
 *   consumer: x_sumsq given (no residual, no next norm): x is the producer's
 *     xg_out and x_sumsq its sumsq_out ([M][K/16], K = 1024 or 2048); the
 *     result is t2i_w4a16_linear_tiles with norm_weight, eps: the
 *     products of bf16(x_raw * norm_weight) scaled by bf16(1/sqrt(mean + eps)),
 *     the mean taken from x_sumsq (the same bits up to the order in which the
 *     row's squares are summed).
 * Decode row counts only; the plan must be one of the chained forms:
 * t2i_w4a16_chain_supported(M, K, N, role) says which (role 0 producer, 1
 * consumer, 2 paired consumer), else the call returns T2I_ERR_SHAPE.  No
 * counterpart in the reference: its fused RMSNorm + projection operators
 * (Q4NXFusedQKVProjection / Q4NXFusedUpGateProjection) do the norm in the consumer.
 */
int t2i_w4a16_linear_tiles_chain(const uint16_t* x, int32_t M, const float* x_sumsq, float eps,
                                 const int32_t* qweight, const int32_t* tiles, const int32_t* qzeros,
                                 const uint16_t* scales, int32_t K, int32_t N, int32_t group_size,
                                 int32_t epilogue, const uint16_t* residual, uint16_t* y0, uint16_t* y1,
                                 const uint16_t* next_norm_weight, uint16_t* xg_out, float* sumsq_out,
                                 void* stream);
int t2i_w4a16_chain_supported(int32_t M, int32_t K, int32_t N, int32_t role);

/* ---------------------------------------------------------------------------
 * Weighted RMSNorm over rows of H: y = bf16(bf16(x * bf16(rsqrt(mean(x^2)+eps))) * w).
 * tokens != NULL: x rows are gathered from the bf16 table `x` ([V, H]) by token id
 * and the gathered rows are also written to x_out (the residual stream); an id
 * outside [0, V) gathers a zero row.  V is ignored when tokens == NULL.
 * argmax_keys != NULL: its M uint64 entries are zeroed (the lm_head argmax reduction
 * starts from zero).
 * Replaces: torch2iron/operators/rms_norm (RMSNorm, weighted), quantized_qwen3/model.py:172-181,
 *           and the host embedding of quantized_qwen3/qwen_npu.py:182-185.
 */
int t2i_rmsnorm(const uint16_t* x, const int32_t* tokens, int32_t V, int32_t M, int32_t H,
                const uint16_t* weight, float eps, uint16_t* x_out, uint16_t* y,
                uint64_t* argmax_keys, void* stream);

/* ---------------------------------------------------------------------------
 * GQA decode attention with the current token folded in.
 * qkv bf16 [B, (Hq + 2*Hkv)*D] is the raw fused q|k|v projection of the current token.
 * Per sequence b (position p = positions[b]):
 *   q, k <- per-head RMSNorm (q_norm / k_norm weights, eps) then RoPE from the bf16
 *           cos/sin table rope[p] ([ctx_cap, D], cos at even, sin at odd columns);
 *           rope_style 0 = halves (i, i+D/2), 1 = interleaved (2i, 2i+1);
 *   k_cache[b][h][p] <- k, v_cache[b][h][p] <- v;
 *   ctx[b][hq*D:] = softmax(q . K[0..p]^T / sqrt(D)) . V[0..p]   (fp32 softmax, bf16 out).
 * A position outside [0, ctx_cap) writes no cache slot and yields a zero context row.
 * Caches are bf16 [B, Hkv, ctx_cap, D].  D = 128; Hq % Hkv == 0; Hq/Hkv <= 8.
 * Replaces: torch2iron/operators/rms_norm_rope (RMSNormRoPE), copy_present_packet_kv
 *           (CopyPresentPacketKV) and llama_chunked_attention (LlamaChunkedAttention),
 *           as wired per layer in quantized_qwen3/batch_decode_fused.py:426-463.
 */
size_t t2i_decode_attention_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t ctx_cap);
int t2i_decode_attention(const uint16_t* qkv, const int32_t* positions, int32_t B,
                         int32_t Hq, int32_t Hkv, int32_t D,
                         const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                         const uint16_t* rope, int32_t rope_style,
                         uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap,
                         uint16_t* ctx, void* workspace, size_t workspace_bytes,
                         void* stream);

/* The same attention on q / k / v that are normalised and rotated already (the
 * reference's runlist runs RMSNormRoPE on them first): q bf16 [B, Hq*D], k and v
 * bf16 [B, Hkv*D].  Per sequence b: k_cache[b][h][p] <- k, v_cache[b][h][p] <- v,
 * ctx as t2i_decode_attention; no norm weights and no RoPE table.  Workspace as
 * t2i_decode_attention (t2i_decode_attention_workspace_bytes).
 * Replaces: torch2iron/operators/copy_present_packet_kv (CopyPresentPacketKV) and
 *           llama_chunked_attention (LlamaChunkedAttention), the per-row pair of
 *           quantized_qwen3/batch_decode_fused.py:445-479 (the KV cache here is
 *           contiguous [B, Hkv, ctx_cap, D], not the 64-slot packet layout).
 */
int t2i_decode_attention_prepared(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                  const int32_t* positions, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                                  uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap, uint16_t* ctx,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Standalone elementwise operators of the reference's batch-decode runlist.  The
 * decode layer folds each into a neighbouring kernel; these run a runlist written
 * for the NPU entry for entry.  Outputs may alias inputs.
 *
 * t2i_rmsnorm_rope: rows of `cols` values; y = RoPE(RMSNorm(x) * weight), row r
 * rotated by angle row r / (rows / angle_rows) of `angles` (bf16 [angle_rows,
 * cols], cos at even, sin at odd columns), rounded as t2i_decode_attention's
 * prologue.  rope_style 0 = halves (i, i + cols/2), 1 = interleaved.  cols even,
 * at most 1024; angle_rows divides rows.
 * Replaces: torch2iron/operators/rms_norm_rope (RMSNormRoPE, op.py:20-96,
 *           kernel.cc:39-67).
 *
 * t2i_silu_mul: out = bf16(bf16(silu(left)) * right) over n values (n % 8 == 0),
 * the SwiGLU epilogue's rounding.
 * Replaces: torch2iron/operators/silu_mul (SiLUMul, op.py:20-79).
 *
 * t2i_residual_add_rmsnorm: x_out = bf16(x + update), y = t2i_rmsnorm(x_out,
 * weight, eps) bit for bit; M rows of H.
 * Replaces: torch2iron/operators/residual_add_rms_norm (ResidualAddRMSNorm,
 *           op.py:19-93).
 */
int t2i_rmsnorm_rope(const uint16_t* x, int32_t rows, int32_t cols, const uint16_t* weight,
                     const uint16_t* angles, int32_t angle_rows, float eps, int32_t rope_style,
                     uint16_t* y, void* stream);
int t2i_silu_mul(const uint16_t* left, const uint16_t* right, int64_t n, uint16_t* out, void* stream);
int t2i_residual_add_rmsnorm(const uint16_t* x, const uint16_t* update, int32_t M, int32_t H,
                             const uint16_t* weight, float eps, uint16_t* x_out, uint16_t* y, void* stream);

/* ---------------------------------------------------------------------------
 * The front of the decode layer in one cooperative launch: the input RMSNorm +
 * fused q|k|v projection of t2i_w4a16_rmsnorm_linear (norm_weight != NULL; with
 * NULL, x is taken as already normalised, as t2i_w4a16_linear), then the
 * attention of t2i_decode_attention on those q, k, v rows (q/k RMSNorm, RoPE,
 * KV-cache write at positions[b], GQA attention), ctx bf16 [B, Hq * D].  The
 * projection's weight holds q, k, v columns (N = (Hq + 2 Hkv) * D); K is the
 * hidden size.  The projection is bit-identical to the standalone call; the
 * attention splits the context differently, so ctx may differ from
 * t2i_decode_attention's by rounding.  1 <= B <= 16, Hq / Hkv in {1, 2}, D = 128,
 * B * Hkv no more than the device's CUs.  One 16-wave workgroup per CU, all
 * resident at once: launches of this call must not run concurrently with other
 * work on the device.  The workspace (t2i_qkv_attention_workspace_bytes) must be
 * zero-filled before its first use and not shared by calls that overlap in
 * time; a wait inside the launch that times out sets the 32-bit word at
 * t2i_qkv_attention_error_offset() of the workspace (zero otherwise).
 * Replaces: the per-layer front of quantized_qwen3/batch_decode_fused.py:426-479
 *           (RMSNorm, query and key/value GEMMs, RMSNormRoPE, CopyPresentPacketKV,
 *           LlamaChunkedAttention), fast_qwen3/operators/qwen3_layer_fused/op.py:18-50.
 */
size_t t2i_qkv_attention_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv);
size_t t2i_qkv_attention_error_offset(int32_t B, int32_t Hq, int32_t Hkv);
int t2i_qkv_attention(const uint16_t* x, int32_t B, const uint16_t* norm_weight, float eps,
                      const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales, int32_t K,
                      int32_t group_size, const int32_t* positions, int32_t Hq, int32_t Hkv, int32_t D,
                      const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* rope, int32_t rope_style,
                      uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap, uint16_t* ctx,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Every decoder layer of one decode step in one cooperative launch.
 * Per layer l (weights and caches from layers[l], a device array of n_layers
 * entries): RMSNorm + q|k|v projection (layer 0 takes xn0, already normalised),
 * the attention of t2i_decode_attention (q/k RMSNorm, RoPE, KV write at
 * positions[b]), o_proj + residual, RMSNorm + paired gate/up + SwiGLU, down +
 * residual.  x bf16 [B, hidden] is the residual stream: the embedding rows in,
 * the last layer's output out.  Weights as the t2i_w4a16_* calls take them
 * (gate_up interleaved as for t2i_w4a16_gate_up, N = 2 * intermediate); norm
 * weights bf16; caches bf16 [B, Hkv, ctx_cap, D] per layer.
 * Every linear gives the bits the standalone calls give on the same input; the
 * attention is t2i_qkv_attention's (the context may differ from
 * t2i_decode_attention's by rounding).  Supported: 1 <= B <= 16, Hq / Hkv in
 * {1, 2}, D = 128, group 128, and shapes whose decode-linear plans are the
 * 16-wave tiles (t2i_decode_step_workspace_bytes returns 0 otherwise; Qwen3-0.6B
 * fits).  One 16-wave workgroup per CU, all resident: launches must not run
 * concurrently with other work on the device.  The workspace must be
 * zero-filled before first use and not shared by calls that overlap in time; a
 * wait that times out sets the error word (t2i_decode_step_offset, region 4).
 * Replaces: the whole-step runlist of quantized_qwen3/batch_decode_fused.py:426-539
 *           compiled into one ELF (batch_decode_fused.py:556-588) and run as one
 *           dispatch (FusedFullELFCallable.__call__, fusion.py:821-840), lm_head
 *           excepted.
 */
typedef struct {
  const int32_t* qkv_qweight;
  const int32_t* qkv_qzeros;
  const uint16_t* qkv_scales;
  const int32_t* o_qweight;
  const int32_t* o_qzeros;
  const uint16_t* o_scales;
  const int32_t* gate_up_qweight;
  const int32_t* gate_up_qzeros;
  const uint16_t* gate_up_scales;
  const int32_t* down_qweight;
  const int32_t* down_qzeros;
  const uint16_t* down_scales;
  const uint16_t* input_norm;
  const uint16_t* post_attention_norm;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  uint16_t* k_cache;
  uint16_t* v_cache;
} t2i_decode_layer;

size_t t2i_decode_step_workspace_bytes(int32_t B, int32_t n_layers, int32_t hidden, int32_t intermediate,
                                       int32_t Hq, int32_t Hkv);
/* Byte offset in the workspace of (after a launch, as 32-bit words with the bf16
 * bits in the low half): 0 the per-layer contexts [L, B, Hq * D], 1 the residual
 * stream after each layer's attention [L, B, hidden], 2 the SwiGLU outputs
 * [L, B, intermediate], 3 the residual stream between layers [L - 1, B, hidden];
 * 4 the 32-bit error word; 0 for an unsupported shape or region.  (The first
 * B * (Hq + 2 Hkv) * D 64-bit words hold the last layer's q|k|v projection, bf16
 * bits in the low 16 bits.) */
size_t t2i_decode_step_offset(int32_t B, int32_t n_layers, int32_t hidden, int32_t intermediate,
                              int32_t Hq, int32_t Hkv, int32_t region);
int t2i_decode_step(const t2i_decode_layer* layers, int32_t n_layers, const uint16_t* xn0, uint16_t* x,
                    int32_t B, int32_t hidden, int32_t intermediate, int32_t Hq, int32_t Hkv, int32_t D,
                    int32_t group_size, const int32_t* positions, const uint16_t* rope, int32_t rope_style,
                    int32_t ctx_cap, float eps, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free variant of t2i_decode_attention.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The chunk states live in a library-held scratch array of
 * T2I_DECODE_ATTENTION_SCRATCH_BYTES per device (held until the process ends):
 * at most 8192 (sequence, kv head) pairs and 16 MiB minus 32 KiB of chunk
 * states, else T2I_ERR_WORKSPACE.  Arguments and results as
 * t2i_decode_attention.  Every call on one GPU shares that GPU's scratch:
 * calls that overlap in time on one GPU (different streams) race. */
#define T2I_DECODE_ATTENTION_SCRATCH_BYTES ((size_t)16 << 20)
int t2i_decode_attention_noalloc(const uint16_t* qkv, const int32_t* positions, int32_t B,
                                 int32_t Hq, int32_t Hkv, int32_t D,
                                 const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                 const uint16_t* rope, int32_t rope_style,
                                 uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap,
                                 uint16_t* ctx, void* stream);

/* ---------------------------------------------------------------------------
 * Prompt (prefill) attention, every prompt row of B sequences at once.  Rows of
 * qkv are b * T + t for prompt token t of sequence b at position p0 + t.
 *
 * t2i_prefill_qk_rope_kv: per-head q/k RMSNorm + RoPE (as t2i_decode_attention's
 * prologue) of every row; q_out bf16 [B, Hq, T, D]; k and v written to
 * k_cache / v_cache [B, Hkv, ctx_cap, D] at positions p0 .. p0 + T - 1.
 *
 * t2i_prefill_attention: causal GQA attention of those rows over cache slots
 * 0 .. p0 + t (slots before p0 hold an earlier prompt chunk); fp32 scores and
 * online softmax, softmax weights rounded to bf16 for the product with V (as
 * quantized_qwen3/model.py:277 in bf16 compute); out bf16 [B * T, Hq * D].
 * D = 128; Hq / Hkv in {1, 2, 4, 8}; p0 + T <= ctx_cap.
 * Replaces: the prompt pass of quantized_qwen3/model.py:453-478 (causal mask
 *           271-275) and the NPU prefill runtime quantized_qwen3/prefill_runtime.py:95-164
 *           with torch2iron/operators/llama_chunked_prefill_attention.
 */
int t2i_prefill_qk_rope_kv(const uint16_t* qkv, int32_t B, int32_t T, int32_t p0, int32_t Hq, int32_t Hkv,
                           int32_t D, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                           const uint16_t* rope, int32_t rope_style, uint16_t* q_out,
                           uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap, void* stream);
int t2i_prefill_attention(const uint16_t* q, int32_t B, int32_t T, int32_t p0, int32_t Hq, int32_t Hkv,
                          int32_t D, const uint16_t* k_cache, const uint16_t* v_cache, int32_t ctx_cap,
                          uint16_t* out, void* stream);

/* ---------------------------------------------------------------------------
 * The prompt pass's q|k|v projection and its q/k RMSNorm + RoPE + KV-cache write
 * in one launch: exactly t2i_w4a16_linear(x, B*T rows, the fused q|k|v weight,
 * N = (Hq + 2*Hkv) * D) followed by t2i_prefill_qk_rope_kv on its output (the
 * same bits in q_out and the caches), without writing or reading back the
 * projection.  Each 64-row x 128-column tile of the prompt GEMM is one head, and
 * its epilogue runs the prep on it.  B*T >= 512 (the prompt GEMM's rows), D = 128;
 * every pointer 16-byte aligned.
 * Replaces: the q|k|v projection and the per-head norm / RoPE / cache write of the
 *           prompt pass (quantized_qwen3/model.py:240-253 per token, and
 *           quantized_qwen3/prefill_runtime.py:95-164 on the NPU).
 */
int t2i_prefill_qkv_rope_kv(const uint16_t* x, int32_t B, int32_t T, int32_t p0, const int32_t* qweight,
                            const int32_t* qzeros, const uint16_t* scales, int32_t K, int32_t group_size,
                            int32_t Hq, int32_t Hkv, int32_t D, const uint16_t* q_norm, const uint16_t* k_norm,
                            float eps, const uint16_t* rope, int32_t rope_style, uint16_t* q_out,
                            uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap, void* stream);

/* ---------------------------------------------------------------------------
 * Row group sums handed from the kernel that writes a prompt GEMM's input to the
 * GEMM.  The prompt GEMM's zero-point term needs, for every row and 128-wide k
 * group, the sum of the row's bf16 values over the group; given them, it skips
 * the all-ones products that otherwise form them (a third of its matrix-core
 * work).  Sums are fp32 and group-major: [K / 128][rows] (sum_parts = 1), or two
 * sums per group over its 64-wide halves, [K / 64][rows] (sum_parts = 2), so that
 * one group's sums for a tile of rows are contiguous; every pointer to sums is
 * 4-byte aligned.  The outputs are those of the plain entry points up to fp32
 * rounding of the sums.  No counterpart in the reference (its NPU kernels apply
 * the zero point per weight): they serve the prompt pass only.
 *
 * t2i_rmsnorm_sums: t2i_rmsnorm (no argmax keys) that also writes y_sums, the
 *   group sums of y; H % 128 == 0.
 * t2i_prefill_attention_sums: t2i_prefill_attention that also writes out_sums
 *   [Hq][B * T], each head's sum of its bf16 context values (one group of the
 *   o_proj's k when D = 128).
 * t2i_w4a16_linear_sums / t2i_w4a16_gate_up_sums / t2i_prefill_qkv_rope_kv_sums:
 *   the plain entry points, taking x_sums (ignored below the prompt GEMM's rows).
 *   gate_up_sums also takes x_sums = NULL (the GEMM then forms them); with
 *   swiglu != 0 it also writes y_sums (may be NULL), the half-group
 *   sums of h, [N / 128][M] (sum_parts = 2 for the down projection); it needs the
 *   prompt GEMM (M >= 512, N % 128 == 0) and fails otherwise.
 */
int t2i_rmsnorm_sums(const uint16_t* x, const int32_t* tokens, int32_t V, int32_t M, int32_t H,
                     const uint16_t* weight, float eps, uint16_t* x_out, uint16_t* y, float* y_sums,
                     void* stream);
int t2i_prefill_attention_sums(const uint16_t* q, int32_t B, int32_t T, int32_t p0, int32_t Hq, int32_t Hkv,
                               int32_t D, const uint16_t* k_cache, const uint16_t* v_cache, int32_t ctx_cap,
                               uint16_t* out, float* out_sums, void* stream);
int t2i_w4a16_linear_sums(const uint16_t* x, const float* x_sums, int32_t sum_parts, int32_t M,
                          const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales, int32_t K,
                          int32_t N, int32_t group_size, const uint16_t* residual, uint16_t* y, void* stream);
int t2i_w4a16_gate_up_sums(const uint16_t* x, const float* x_sums, int32_t sum_parts, int32_t M,
                           const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales, int32_t K,
                           int32_t N, int32_t group_size, int32_t swiglu, uint16_t* y0, uint16_t* y1,
                           float* y_sums, void* stream);
int t2i_prefill_qkv_rope_kv_sums(const uint16_t* x, const float* x_sums, int32_t B, int32_t T, int32_t p0,
                                 const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                                 int32_t K, int32_t group_size, int32_t Hq, int32_t Hkv, int32_t D,
                                 const uint16_t* q_norm, const uint16_t* k_norm, float eps, const uint16_t* rope,
                                 int32_t rope_style, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                                 int32_t ctx_cap, void* stream);

/* ---------------------------------------------------------------------------
 * Tied bf16 lm_head with a fused greedy argmax.
 * logits[m][v] = sum_k h[m][k] * E[v][k] in fp32 (E bf16 [V, K], K % 64 == 0, V % 16 == 0).
 * argmax_keys (uint64 [M], zeroed beforehand, e.g. by t2i_rmsnorm) receives
 * ordered(max logit) << 32 | (0xFFFFFFFF - index): the first index of the maximum
 * wins ties, as torch.argmax.  logits (nullable) receives fp32 logits [M, V].
 * Replaces: quantized_qwen3/operators/w4a16_gemm/op.py:337-399 (W4A16NShardGEMM lm_head)
 *           and the host argmax of quantized_qwen3/qwen_npu.py:321.
 */
int t2i_lm_head_argmax(const uint16_t* h, int32_t M, const uint16_t* E, int32_t V,
                       int32_t K, float* logits, uint64_t* argmax_keys, void* stream);

/* ---------------------------------------------------------------------------
 * The final RMSNorm and the lm_head in one launch: exactly t2i_rmsnorm(x,
 * norm_weight, eps) followed by t2i_lm_head_argmax on the normalised rows (the
 * same bits in logits and argmax_keys), with the norm applied by every workgroup
 * to its staged copy of the rows.  K must be a power of two in [64, 4096];
 * argmax_keys zeroed beforehand (e.g. by the step's embedding-gather t2i_rmsnorm).
 * Replaces: logits = self.lm_head(self.norm(x)) of quantized_qwen3/model.py:477.
 */
int t2i_rmsnorm_lm_head_argmax(const uint16_t* x, int32_t M, const uint16_t* norm_weight, float eps,
                               const uint16_t* E, int32_t V, int32_t K, float* logits,
                               uint64_t* argmax_keys, void* stream);

/* ---------------------------------------------------------------------------
 * Greedy bookkeeping between decode steps, on the device:
 * tokens[b] = index decoded from argmax_keys[b]; history[b*hist_cap + step[0]] = tokens[b];
 * positions[b] += 1; step[0] += 1 (by one thread after all rows).  Lets a captured
 * decode step be replayed without host work.
 * Replaces: the host loop of quantized_qwen3/qwen_npu.py:318-325.
 */
int t2i_greedy_advance(const uint64_t* argmax_keys, int32_t B, int32_t* tokens,
                       int32_t* positions, int32_t* history, int32_t hist_cap,
                       int32_t* step, void* stream);

/* Teacher-forced prompt step: positions[b] += 1; tokens[b] = prompt[b*P + positions[b]]
 * while positions[b] < P.  prompt is int32 [B, P].
 * Replaces: the per-sequence prefill loop of quantized_qwen3/qwen_npu.py:309-315
 *           (prompt consumed one position at a time through the decode path). */
int t2i_prompt_advance(const int32_t* prompt, int32_t B, int32_t P, int32_t* tokens,
                       int32_t* positions, void* stream);

/* ---------------------------------------------------------------------------
 * Measurement helper, no counterpart in the reference: the HBM read ceiling that
 * a linear's bandwidth is compared with.  Reads `bytes` (a positive multiple of
 * 16) from src with 16-byte loads, loads_per_thread (1, 2, 4 or 8) per thread in
 * 256-thread workgroups, and writes the XOR of each wave's 32-bit words to out:
 * t2i_stream_read_out_words(bytes, loads_per_thread) words, word w covering the
 * 64 * loads_per_thread 16-byte words of wave w (0 when the arguments are invalid).
 */
int64_t t2i_stream_read_out_words(size_t bytes, int32_t loads_per_thread);
int t2i_stream_read(const void* src, size_t bytes, int32_t loads_per_thread, uint32_t* out,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* T2I_HIP_H */
