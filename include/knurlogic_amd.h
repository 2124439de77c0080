/*
 * knurlogic_amd -- C ABI of the MI355X (gfx950) quantized-weight kernels.
 *
 * The drop-in boundary for the reference's quantized-weight hot path.  In
 * the reference (Knurlogic 0.1.9) that path sits behind mlx's Python ops
 * (mx.quantize / mx.dequantize / mx.quantized_matmul / mx.gather_qmm, mlx
 * 0.32.3 pinned at pyproject.toml:32) and the reference's own 8-bit-KV decode
 * kernel (src/knurlogic/engine/kvattn.py:256-291).  Each entry point below
 * replaces one of those; the Python mirror (knurlogic_amd/ops.py) binds
 * them with ctypes.
 *
 * Conventions
 *   - Every compute entry point returns 0 on success or a negative code
 *     (-1 bad argument, -2 HIP error, -3 workspace too small) and leaves a
 *     message for kmi_last_error() (thread-local).
 *   - The caller allocates every input, output and workspace buffer (device
 *     memory); the library never allocates or frees.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *     and is stream-ordered: nothing is synchronised.
 *   - dtype codes: 0 bfloat16, 1 float16, 2 float32.
 *   - Packed affine layout (mlx's): element j of a row lives in uint32 word
 *     j / (32/bits) at bit offset (j % (32/bits)) * bits; scales and biases
 *     hold one value per group of `group_size` consecutive elements of a row.
 */
#ifndef KNURLOGIC_AMD_H
#define KNURLOGIC_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KMI_ABI_VERSION 1

/* Message of the last failing call on this thread ("" if none). */
const char* kmi_last_error(void);

/* KMI_ABI_VERSION of the built library. */
int kmi_abi_version(void);

/*
 * mx.quantize(w, group_size, bits, mode="affine") over the last axis of a
 * row-major [rows, cols] tensor.  Replaces mlx's affine quantizer as called
 * at src/knurlogic/engine/kvquant.py:46-47 (KV append) and
 * src/knurlogic/engine/families/glm5/architecture/glm5_next/_mlx_vlm/models/
 * switch_layers.py:38-48 (weights).
 *   w       [rows, cols] of `dtype`, 16-byte aligned
 *   wq      [rows, cols*bits/32] uint32 out
 *   scales, biases [rows, cols/group_size] of `dtype` out
 * bits in {2, 3, 4, 5, 6, 8} (3, 5 and 6-bit codes back to back in the row's
 * little-endian bit stream, mlx's packing of those widths); group_size in
 * {32, 64, 128}.
 */
int kmi_quantize_affine(const void* w, int dtype, int64_t rows, int64_t cols,
                        int group_size, int bits, uint32_t* wq, void* scales,
                        void* biases, void* stream);

/*
 * Quantize-on-append for a quantized KV cache: the reference's
 * QuantKVCache / BatchQuantKVCache.update_and_fetch writes
 * mx.quantize(keys) into slab slots prev .. prev+S
 * (src/knurlogic/engine/kvquant.py:136-155,214-234).  x [B, H, S, D]
 * contiguous (dtype), 16-byte aligned, quantized along D in groups of
 * group_size (the same arithmetic as kmi_quantize_affine, bit for bit),
 * written to slots
 * n = pos .. pos+S-1 of a cache triple: wq u32 [B, H, capacity, D*bits/32],
 * scales / biases [B, H, capacity, D/group_size] (dtype), each possibly a
 * strided view with a contiguous last axis.  strides[6]: element strides
 * (b, h, n) of wq, then (b, h, n) shared by scales and biases.
 */
int kmi_kv_quantize_append(const void* x, int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                           int group_size, int bits, uint32_t* wq, void* scales, void* biases,
                           const int64_t* strides, int64_t pos, int64_t capacity, void* stream);

/*
 * Keys and values of one update_and_fetch in one launch (the two
 * mx.quantize writes of kvquant.py:153-156): as kmi_kv_quantize_append for
 * k [B, H, S, Dk] into the K triple and v [B, H, S, Dv] into the V triple,
 * same dtype, group and bits; each triple with its own strides[6].
 */
int kmi_kv_quantize_append_kv(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t S,
                              int64_t Dk, int64_t Dv, int group_size, int bits, uint32_t* k_wq, void* k_scales,
                              void* k_biases, const int64_t* k_strides, uint32_t* v_wq, void* v_scales,
                              void* v_biases, const int64_t* v_strides, int64_t pos, int64_t capacity,
                              void* stream);

/*
 * mx.quantize(w, group_size=32, mode="mxfp4" | "mxfp8") over [rows, cols]:
 * per group of 32 the OCP shared exponent X = floor(log2 max|w|) - emax
 * (emax 2 for E2M1, 8 for E4M3) stored as the E8M0 byte X + 127 (an
 * all-zero group: 0), elements w / 2^X rounded to the nearest code (ties to
 * even) and saturated, the sign of w kept on every code (-0 included):
 * the OCP MX v1.0 conversion.  mlx's own quantizer is not in the
 * reference tree, so its tie, saturation and zero-sign behaviour is not
 * pinned; the reference's mxfp4 checkpoint
 * (tests/support/goldens/deepseek_v4_tiny) re-quantizes to itself, which
 * checks the shared exponent only.  wq [rows, cols*bits/32], scales uint8
 * [rows, cols/32].
 */
int kmi_quantize_mx(const void* w, int dtype, int64_t rows, int64_t cols, int mode, uint32_t* wq,
                    uint8_t* scales, void* stream);

/*
 * mx.dequantize(w, scales, mode="mxfp4" | "mxfp8") over [rows, cols]: element
 * codes E2M1 (mode 1, 4 bits) or E4M3 (mode 2, 8 bits) packed as mlx packs
 * 4 / 8-bit codes, times 2^(e - 127) for the uint8 E8M0 scale e of each group
 * of 32 (scales [rows, cols/32]) -- the scaled modes the reference's loader
 * maps layers without biases to (src/knurlogic/engine/model/packed.py:20,
 * load_model.py:153-173).  out in out_dtype.
 */
int kmi_dequantize_mx(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t cols, int mode,
                      void* out, int out_dtype, void* stream);

/*
 * mx.dequantize(wq, scales, biases, group_size, bits, mode="affine",
 * dtype=out_dtype), as called at src/knurlogic/engine/kvquant.py:50-51.
 *   rounding 0: out = T(T(scale*q) + bias)  (op-by-op, the default)
 *   rounding 1: out = T(fma(scale, q, bias))
 * bits in {2, 3, 4, 5, 6, 8}, codes packed as kmi_quantize_affine writes them.
 */
int kmi_dequantize_affine(const uint32_t* wq, const void* scales, const void* biases,
                          int scale_dtype, int64_t rows, int64_t cols, int group_size,
                          int bits, void* out, int out_dtype, int rounding, void* stream);

/*
 * mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits)
 * -- nn.QuantizedLinear's op (swapped in at
 * src/knurlogic/engine/model/load_model.py:124-144; wrapped at
 * src/knurlogic/engine/matmul_padding.py:94-105):
 *   y[M, N] = x[M, K] @ What[N, K]^T,  What = scale * q + bias,
 * fp32 accumulation, y rounded once to `dtype`.  x, scales, biases, y share
 * `dtype`.  Decode shapes (M <= 16) run the streaming GEMV kernel, larger M
 * the LDS-tiled MFMA GEMM.  Each output row depends only on its own input row.
 * `workspace` (kmi_qmm_workspace_bytes) holds split-K partials; it may be
 * NULL when that size is 0.
 */
int kmi_qmm(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w,
            const void* scales, const void* biases, int dtype, int group_size,
            int bits, void* y, void* workspace, size_t workspace_bytes, void* stream);

size_t kmi_qmm_workspace_bytes(int64_t M, int64_t K, int64_t N, int group_size, int bits);

/*
 * mx.quantized_matmul(x, w, scales, transpose=True, group_size=32, bits,
 * mode="mxfp4" | "mxfp8") -- nn.QuantizedLinear of the loader's microscaled
 * layers (src/knurlogic/engine/model/load_model.py:153-173):
 *   y[M, N] = x[M, K] @ What[N, K]^T,  What = code * 2^(e - 127),
 * codes E2M1 (mode 1, 4 bits, 8 per uint32) or E4M3 (mode 2, 8 bits, 4 per
 * uint32), one uint8 E8M0 scale e per 32 inputs (scales [N, K/32]), no
 * biases; fp32 accumulation, y rounded once to bf16 (x and y bf16).  Up to
 * 64 rows with K a multiple of 64 run kmi_qmm's decode kernels (M = 1: the
 * streaming GEMV; 2..16 rows with K a multiple of 256: the direct-to-LDS
 * MFMA kernel; else the MFMA GEMV), anything else kmi_qmm_batched.  Each
 * output row depends only on its own input row.  `workspace`
 * (kmi_qmm_mx_workspace_bytes) holds split-K partials; it may be NULL when
 * that size is 0.
 */
int kmi_qmm_mx(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w, const uint8_t* scales,
               int dtype, int mode, void* y, void* workspace, size_t workspace_bytes, void* stream);

size_t kmi_qmm_mx_workspace_bytes(int64_t M, int64_t K, int64_t N, int mode);

/*
 * kmi_qmm without a workspace argument, allocating nothing: no counterpart
 * in the reference.  It is for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops that forbid hipMalloc).  The
 * same kernels as kmi_qmm, with the split-K partials in a device array of
 * KMI_QMM_SCRATCH_BYTES that the library holds on every GPU it runs on
 * until the process ends (its address is looked up once per device, on the
 * first call with that device current).  Shapes whose partials need more
 * (kmi_qmm_workspace_bytes > KMI_QMM_SCRATCH_BYTES) are refused with -1.
 * The caller still allocates x and y.  All calls on one GPU share its
 * array: calls that overlap on one GPU (two streams or threads) race.
 */
#define KMI_QMM_SCRATCH_BYTES (32u << 20)
size_t kmi_qmm_noalloc_scratch_bytes(void);
int kmi_qmm_noalloc(const void* x, int64_t M, int64_t K, int64_t N, const uint32_t* w,
                    const void* scales, const void* biases, int dtype, int group_size,
                    int bits, void* y, void* stream);

/*
 * mx.gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices,
 * transpose=True, group_size, bits, sorted_indices) -- QuantizedSwitchLinear's
 * op (src/knurlogic/engine/families/glm5/architecture/glm5_next/_mlx_vlm/
 * models/switch_layers.py:71-86), with the broadcast index pairs already
 * flattened by the caller:
 *   for p < P, m < M:  y[p, m, :] = x[lhs[p], m, :] @ What[rhs[p]]^T
 *   x [X, M, K], w [E, N, K*bits/32], scales/biases [E, N, K/group_size],
 *   lhs/rhs [P] int32, y [P, M, N].
 * Rows are grouped by expert on the GPU (counting sort into `workspace`), so
 * each routed expert's packed weights are streamed once per call whether or
 * not `sorted_indices` holds; the flag is accepted for signature parity.
 */
int kmi_gather_qmm(const void* x, int64_t X, int64_t M, int64_t K, const uint32_t* w,
                   const void* scales, const void* biases, int64_t E, int64_t N,
                   const int32_t* lhs, const int32_t* rhs, int64_t P, int dtype,
                   int group_size, int bits, int sorted_indices, void* y,
                   void* workspace, size_t workspace_bytes, void* stream);

size_t kmi_gather_qmm_workspace_bytes(int64_t P, int64_t M, int64_t E, int64_t K,
                                      int64_t N, int group_size, int bits);

/*
 * 8-bit-KV decode attention: the reference's kvattn.decode_sdpa
 * (src/knurlogic/engine/kvattn.py:256-291, kernels :78-183) over the
 * quantized cache triples that kvquant's caches hold
 * (src/knurlogic/engine/kvquant.py:60-63):
 *   q [B, H, L, D] contiguous (q_dtype); out [B, H, L, D] (q_dtype);
 *   K = (kw u32 [B, Hk, N, D/4], ks, kb [B, Hk, N, D/group]), V likewise,
 *   each of the six possibly a strided view (slab[..., :N, :]): strides[18]
 *   holds the element strides (b, h, n) of kw, ks, kb, vw, vs, vb in that
 *   order; the last axis is contiguous.  scale_dtype: dtype of ks/kb/vs/vb.
 *   Query head h reads KV head h / (H/Hk); q is pre-multiplied by `scale`.
 *   mask: [B, L, N] uint8 (1 = visible) or NULL; causal (L > 1): row l sees
 *   keys n <= N - L + l.  A row that sees no key is 0.
 * D in {128, 256, 384, 512}; group divides D and is a multiple of 16 (the
 * reference takes multiples of D/32 -- kvattn.py:221-222 -- which adds
 * groups of 4 and 8 at D = 128 and of 8 at D = 256, sizes mlx's quantize
 * does not make); (H/Hk)*L <= 64; 8-bit only.  `workspace`
 * (kmi_kv8_workspace_bytes) holds the per-block partials.
 */
int kmi_kv8_decode(const void* q, int q_dtype, int B, int H, int L, int D,
                   const uint32_t* kw, const void* ks, const void* kb,
                   const uint32_t* vw, const void* vs, const void* vb,
                   const int64_t* strides, int scale_dtype, int Hk, int N, int group,
                   float scale, const uint8_t* mask, int causal, void* out,
                   void* workspace, size_t workspace_bytes, void* stream);

size_t kmi_kv8_workspace_bytes(int B, int H, int Hk, int L, int N, int D);

/*
 * mx.quantized_matmul with a batched weight, transpose=True or False: the
 * products of mlx-lm's quantized scaled-dot-product attention
 * (src/knurlogic/engine/families/glm5/architecture/glm5_next/_mlx_vlm/
 * models/base.py:281-297: scores = q K^T, transpose=True; out = P V,
 * transpose=False) and of QuantizedMultiLinear (.../_mlx_vlm/models/
 * mla.py:80-87; transpose=False at .../glm5_next/language.py:760).
 *   for every batch index b (nd <= 4 dimensions of batch_shape):
 *     transpose=1: y[b] = x[b] @ What[b]^T, What[b] [N, K], groups along K
 *     transpose=0: y[b] = x[b] @ What[b],   What[b] [K, N], groups along N
 *   x[b] [M, K] bf16, optionally staged as bf16(x * x_scale) (x_scale = 1:
 *   unchanged), y [batch..., M, N] bf16 with row stride ldy >= N (rows
 *   otherwise contiguous).
 * Strides are in elements (x, scales / biases) or words (w): *_strides[d]
 * for batch dimension d (0 broadcasts), then *_strides[nd] between rows.
 * x rows and batch strides are multiples of 8 elements from a 16-byte
 * aligned base, and each row is read in 16-byte units: the elements up to
 * the next multiple of 8 past K must be readable memory (their values are
 * ignored).  With transpose=1 and 4 or 8 bits the weight rows are 16-byte
 * aligned.  bits: 2, 3, 4, 5, 6 or 8 (3, 5 and 6-bit codes are read from the
 * row's little-endian bit stream, mlx's packing of those widths).
 * mode: 0 affine; 1 mxfp4 (E2M1 codes, bits 4); 2 mxfp8 (E4M3 codes, bits
 * 8) -- both with one E8M0 uint8 scale per 32 elements and no biases
 * (biases may be NULL), the modes of load_model.py:153-173.
 * Gather form (mx.gather_qmm, one batch dimension of P pairs): widx[p] picks
 * the weight / scales of pair p among nw stacked ones (w_strides[0] /
 * s_strides[0] apart), xidx[p] (or p) its x entry among nx (x_strides[0]
 * apart); an index out of range gives a zero output.  Both NULL: the strided
 * batch form (nw, nx unused).
 * The weight tile is dequantized in fp32 and fed to the MFMAs as two bf16
 * parts (exact to 2^-17), fp32 accumulation.  `workspace` (kmi_qmm_batched_workspace_bytes) holds
 * split-K partials; it may be NULL when that size is 0.
 */
size_t kmi_qmm_batched_workspace_bytes(int nd, const int64_t* batch_shape, int64_t M, int64_t K, int64_t N);
int kmi_qmm_batched(const void* x, const int64_t* x_strides, const uint32_t* w, const int64_t* w_strides,
                    const void* scales, const void* biases, const int64_t* s_strides, int nd,
                    const int64_t* batch_shape, int64_t M, int64_t K, int64_t N, int transpose, int dtype,
                    int group_size, int bits, int mode, const int32_t* widx, const int32_t* xidx, int64_t nw,
                    int64_t nx, float x_scale, void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                    void* stream);

/* mask kinds of kmi_masked_softmax */
#define KMI_MASK_NONE 0
#define KMI_MASK_BOOL 1   /* uint8, nonzero = visible; hidden scores become finfo(bf16).min */
#define KMI_MASK_ADD 2    /* bf16 added to the scores (rounded to bf16) */
#define KMI_MASK_CAUSAL 3 /* key j hidden from query row l of L when j > N - L + l */

/*
 * The step between mlx-lm's two quantized attention products
 * (.../_mlx_vlm/models/base.py:285-295): mask, then
 * mx.softmax(scores, precise=True) -- max, exp and sum in fp32, the
 * probabilities rounded to bf16.  Rows of x [R, N] (row stride ldx) are
 * indexed by row_dims[4] (row = ((i0*d1 + i1)*d2 + i2)*d3 + i3, d3 the query
 * length L); mask_strides[4] are the mask's element strides over those four
 * dimensions (0 broadcasts), its last axis contiguous.  Rows of x and out
 * are 16-byte aligned and padded to a multiple of 8 elements (ldx, ldo >=
 * N rounded up to 8); out's padding is written with zeros.  out may alias x.
 */
int kmi_masked_softmax(const void* x, int64_t ldx, int dtype, const int64_t* row_dims, int64_t N,
                       const void* mask, int mask_kind, const int64_t* mask_strides, void* out, int64_t ldo,
                       void* stream);

/*
 * mlx's nn.Linear for the layers a quantized model keeps unquantized: the
 * Qwen3.5-MoE router gate and shared-expert gate (qwen3_5.py:173-174,186,
 * self.gate(x) / self.shared_expert_gate(x)):
 *   y[M, N] = x[M, K] @ w[N, K]^T            (bias NULL), or
 *   y[M, N] = addmm(bias, x, w^T)            (one rounding of acc + bias[n])
 * fp32 accumulation, y rounded to `dtype` (bfloat16 or float16); x, w, bias
 * and y share it.  K % 8 == 0, x and w contiguous and 16-byte aligned.
 */
int kmi_linear(const void* x, int64_t M, int64_t K, const void* w, int64_t N, const void* bias, int dtype,
               void* y, void* stream);

/*
 * The bias of nn.QuantizedLinear / QuantizedSwitchLinear, added to the
 * rounded product as its own op (switch_layers.py:82-85:
 * x + expand_dims(bias[indices], -2)):
 *   y[r, n] = round(y[r, n] + bias[e, n]),  e = idx[r / rows_per_index]
 * (idx NULL: e = 0; bias [E, N]); rows with e outside [0, E) are left alone.
 * y [rows, N] in place, bfloat16 or float16.
 */
int kmi_add_bias(void* y, int64_t rows, int64_t N, const void* bias, const int32_t* idx, int64_t rows_per_index,
                 int64_t E, int dtype, void* stream);

/*
 * The MoE router of Qwen3.5-MoE's SparseMoeBlock
 * (src/knurlogic/engine/families/qwen/architecture/qwen3_5.py:174-179):
 * probs = softmax(logits) in float32; the top k in descending order (equal
 * probabilities lower expert first); scores = those probabilities
 * renormalized in float32 and rounded to `dtype`.
 *   logits [T, E] of dtype; inds [T, k] int32 out; scores [T, k] dtype out.
 * E <= 1024, k <= min(E, 64).
 */
int kmi_moe_route(const void* logits, int dtype, int64_t T, int E, int k, int32_t* inds,
                  void* scores, void* stream);

/*
 * _SwiGLU (qwen3_5.py:39-40,108-112), SwitchGLU's activation between the
 * gate/up and down projections:
 *   out[r, i] = round(round(silu_f32(gate[r, i])) * up[r, i])
 * gate/up rows have stride `ld` (elements; e.g. the two halves of one
 * stacked gate|up projection); out [rows, I] contiguous.
 */
int kmi_swiglu(const void* gate, const void* up, int64_t ld, int dtype, int64_t rows,
               int64_t I, void* out, void* stream);

/*
 * The weighted combine of the k expert outputs (qwen3_5.py:181-182,
 * (y * scores[..., None]).sum(-2)):
 *   out[t, h] = round(sum_s round(y[t, s, h] * scores[t, s]))
 * y [T, k, H], scores [T, k], out [T, H], all of `dtype`.
 */
int kmi_moe_combine(const void* y, const void* scores, int dtype, int64_t T, int k, int64_t H,
                    void* out, void* stream);

/*
 * SparseMoeBlock's shared expert added to the routed combine
 * (qwen3_5.py:184-187): out[t, h] = round(y[t, h] +
 * round(round(sigmoid_f32(gate[t])) * shared_y[t, h])).
 * y, shared_y, out [T, H]; gate [T] (the shared_expert_gate logit).
 */
int kmi_moe_shared_add(const void* y, const void* gate, const void* shared_y, int dtype, int64_t T,
                       int64_t H, void* out, void* stream);

/*
 * SwitchGLU with Qwen3.5's _SwiGLU, and optionally the weighted combine, in
 * one call: switch_layers.py:172-193 (SwitchGLU.__call__: up, gate,
 * activation, down through gather_qmm) and qwen3_5.py:108-112,181-182.
 *   x [T, H] bf16; inds [T, k] int32 (k <= 8); scores [T, k] bf16 or NULL;
 *   w_gu / s_gu / b_gu: the gate and up projections stacked per expert,
 *     [E, 2I, H*bits/32] / [E, 2I, H/group] (rows 0..I-1 gate, I..2I-1 up);
 *   w_down / s_down / b_down: [E, H, I*bits/32] / [E, H, I/group];
 *   out: [T, H] = round(sum_s round(y[t, s] * scores[t, s])) when scores is
 *     given, else y [T, k, H] (SwitchGLU's own output).
 * Every intermediate rounds where the reference rounds: gate and up outputs,
 * silu, the activation, the down output, each weighted product.  Up to 64
 * (token, slot) pairs run token-major (two kernels, no sort); more group
 * rows by expert (a GPU sort of the pairs into expert tiles).  workspace:
 * kmi_switch_glu_workspace_bytes.
 */
int kmi_switch_glu(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                   const void* scores, const uint32_t* w_gu, const void* s_gu, const void* b_gu,
                   const uint32_t* w_down, const void* s_down, const void* b_down, int64_t E,
                   int dtype, int group_size, int bits, void* out, void* workspace,
                   size_t workspace_bytes, void* stream);

size_t kmi_switch_glu_workspace_bytes(int64_t T, int64_t H, int64_t I, int k, int64_t E,
                                      int group_size, int bits);

/*
 * kmi_switch_glu for experts stored in an OCP microscaled mode -- the
 * loader's mxfp4 / mxfp8 expert layers (src/knurlogic/engine/model/
 * load_model.py:153-173, packed.py:20) behind the same SwitchGLU
 * (switch_layers.py:172-193): mode 1 mxfp4 (E2M1 codes, 8 per uint32),
 * mode 2 mxfp8 (E4M3, 4 per uint32), one uint8 E8M0 scale per 32 inputs,
 * no biases.  w_gu [E, 2I, H*bits/32] and s_gu [E, 2I, H/32] stack gate
 * (rows 0..I-1) and up; w_down [E, H, I*bits/32], s_down [E, H, I/32].
 * Up to 64 (token, slot) pairs run token-major, more grouped by expert,
 * as kmi_switch_glu (workspace: kmi_switch_glu_workspace_bytes with group
 * 32).
 */
int kmi_switch_glu_mx(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                      const void* scores, const uint32_t* w_gu, const uint8_t* s_gu, const uint32_t* w_down,
                      const uint8_t* s_down, int64_t E, int dtype, int mode, void* out, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * SparseMoeBlock's routed experts from the router logits, in one call
 * (qwen3_5.py:174-182): the router of kmi_moe_route (softmax in float32,
 * top-k, renormalized scores in bf16), then kmi_switch_glu with the
 * weighted combine.  logits [T, E] bf16; inds [T, k] int32 and scores
 * [T, k] bf16 are written (the routing, as kmi_moe_route gives it bit for
 * bit); out [T, H] bf16; the weights as kmi_switch_glu takes them.  At
 * decode sizes (up to 64 (token, slot) pairs, E <= 256) the gate/up kernel
 * routes its own token, so the call is two kernel launches; otherwise it
 * routes first, and up to 256 pairs over up to 256 experts the expert
 * kernels form their tiles from the routed experts (no sort launch).
 * k <= 8, E <= 1024.  workspace: kmi_switch_glu_workspace_bytes.
 */
int kmi_moe_experts(const void* x, const void* logits, int64_t T, int64_t H, int64_t I, int k, int64_t E,
                    const uint32_t* w_gu, const void* s_gu, const void* b_gu, const uint32_t* w_down,
                    const void* s_down, const void* b_down, int dtype, int group_size, int bits, void* out,
                    int32_t* inds, void* scores, void* workspace, size_t workspace_bytes, void* stream);

/*
 * VQ codebook-decode expert matmul: VQSwitchLinear, the expert layer VQ
 * artifacts ship in their own model.py (class named at
 * tests/engine/test_deepseek_v4_mtp.py:249,360; code layout of _pack_vq at
 * :206-233), for 8-element vectors and byte or 16-bit indices:
 *   What_e[o, i] = scales[e, o, i / sg] * codebook[codes[e, o, i / 8]][i % 8]
 *   y[p, :] = x[lhs[p]] @ What_{rhs[p]}^T     (lhs NULL: x row p)
 *   x [X, K] bf16; codes [E, N, K/8] uint8 (code_bytes 1) or uint16 (2);
 *   codebook [kc, 8] fp16 (dim must be 8); scales fp16 [E, N] when
 *   scale_group is 0 (one per output channel), else [E, N, K/scale_group];
 *   y [P, N] bf16.  fp32 accumulation; x enters the dot products as fp16.
 */
int kmi_vq_gather_qmm(const void* x, int64_t X, int64_t K, const void* codes, int code_bytes,
                      const void* codebook, int kc, int dim, const void* scales, int scale_group,
                      int64_t E, int64_t N, const int32_t* lhs, const int32_t* rhs, int64_t P,
                      int dtype, void* y, void* stream);

/*
 * The gate and up VQ projections of SwitchGLU with the _SwiGLU epilogue
 * (switch_layers.py:172-193 over VQSwitchLinear; qwen3_5.py:108-112):
 *   act[t*k + s, :] = round(round(silu(round(gate))) * round(up)) for the
 *   expert inds[t, s] and the token row x[t]; x [T, H]; codes_* [E, I, H/8];
 *   scales_* as kmi_vq_gather_qmm; act [T*k, I] bf16.  The gate and up
 *   codebooks may be the same pointer.
 */
int kmi_vq_glu(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
               const void* codes_gate, const void* scales_gate, const void* codebook_gate,
               const void* codes_up, const void* scales_up, const void* codebook_up, int code_bytes,
               int kc, int dim, int scale_group, int64_t E, int dtype, void* act, void* stream);

/*
 * VQ SwitchGLU in one call (switch_layers.py:172-193 over VQSwitchLinear,
 * with qwen3_5.py's _SwiGLU and the SparseMoeBlock combine at
 * qwen3_5.py:181-182): act = the gate/up projections with the SwiGLU
 * epilogue (as kmi_vq_glu), then the down projection per (token, slot) and,
 * when scores [T, k] bf16 is given, the weighted combine
 *   out[t, :] = round(sum_s round(y[t, s, :] * scores[t, s]))  (out [T, H])
 * (as kmi_moe_combine), else out = y [T*k, H].  codes_down [E, H, I/8]; all
 * three projections share code_bytes, kc, dim and scale_group.
 * workspace: kmi_vq_switch_glu_workspace_bytes(T, H, I, k) bytes.
 */
size_t kmi_vq_switch_glu_workspace_bytes(int64_t T, int64_t H, int64_t I, int k);
/*
 * VQSwitchLinear over the bit-packed on-disk code layout of the VQ
 * artifacts (src/knurlogic/engine/families/deepseek/heads/deepseek_v4.py:
 * 36-44,95-129; shipped as K = 2048 entries of dim 2-4 in 11-bit fields,
 * tests/engine/test_deepseek_v4_mtp.py:206-233):
 *   What_e[o, i] = scales[e, o, i / group] * codebook[field(e, o, i / dim)][i % dim]
 *   y[r, :] = x[rows[r]] @ What_{experts[r]}^T      (r < R; rows NULL: x row r / rows_div)
 *   codes [E, N, W] uint32, W = ceil(K / dim / 32) * pack_bits: field j of a
 *   row at bits [j*pack_bits, (j+1)*pack_bits) of the row's words read as
 *   one little-endian bit stream; pack_bits in 8..12 or 16; codebook
 *   [kc, dim] fp16 (dim 2, 4 or 8); scales [E, N, K / group] fp16 with
 *   group >= 32 and group / dim a power of two; x [X, K] bf16, y [R, N] bf16.
 * fp32 accumulation; x enters the dot products as fp16.  The field order
 * within the words is not fixed by the reference tree (its runtime is not
 * vendored): LSB first, as mlx packs sub-byte fields.
 */
int kmi_vq_packed_gather_qmm(const void* x, int64_t X, int64_t K, const uint32_t* codes, int pack_bits,
                             const void* codebook, int kc, int dim, const void* scales, int group, int64_t E,
                             int64_t N, const int32_t* rows, int64_t rows_div, const int32_t* experts, int64_t R,
                             int dtype, void* y, void* stream);

/*
 * The gate and up projections of a packed VQ SwitchGLU with Qwen3.5's
 * _SwiGLU (qwen3_5.py:108-112) in one launch: act[r, :] =
 * round(round(silu(round(x[rows[r]] @ Gate_e^T))) * round(x[rows[r]] @ Up_e^T)),
 * e = experts[r] (rows NULL: x row r / rows_div, e.g. k slots per token);
 * codes / scales / codebooks as kmi_vq_packed_gather_qmm,
 * gate and up [E, I, *] over H inputs; act [R, I] bf16.
 */
int kmi_vq_packed_glu(const void* x, int64_t X, int64_t H, int64_t I, const uint32_t* codes_gate,
                      const void* scales_gate, const void* codebook_gate, const uint32_t* codes_up,
                      const void* scales_up, const void* codebook_up, int pack_bits, int kc, int dim, int group,
                      int64_t E, const int32_t* rows, int64_t rows_div, const int32_t* experts, int64_t R,
                      int dtype, void* act, void* stream);

/*
 * A whole SwitchGLU over packed VQ experts (the artifact model.py's
 * VQSwitchGLU over VQSwitchLinear, named at tests/engine/test_deepseek_v4_mtp.py:
 * 249,360; gate/up/down as switch_layers.py:172-193) in one call, the
 * weighted combine of qwen3_5.py:181-182 when scores [T, k] bf16 are given:
 *   act = SwiGLU over gate / up as kmi_vq_packed_glu (x row = pair / k),
 *   y[p] = act[p] @ Down_{inds[p]}^T, out = combine(y, scores) [T, H] or y [T*k, H].
 * Codes / scales / codebooks as kmi_vq_packed_gather_qmm (gate and up
 * [E, I, *] over H inputs, down [E, H, *] over I).  Up to 16 pairs run per
 * pair (with scores, k <= 8: the down projection token-major with the
 * combine in its epilogue, the same bits as the separate combine); more
 * are grouped by expert on the GPU (an expert-tile MFMA kernel
 * where the shape allows: dim 2 / 4 / 8, groups of 32 / 64 / 128 inputs,
 * K a multiple of 32 * dim), so pairs that share an expert share its
 * decode.  workspace: kmi_vq_packed_switch_glu_workspace_bytes.
 */
size_t kmi_vq_packed_switch_glu_workspace_bytes(int64_t T, int64_t H, int64_t I, int k);
int kmi_vq_packed_switch_glu(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                             const void* scores, const uint32_t* codes_gate, const void* scales_gate,
                             const void* codebook_gate, const uint32_t* codes_up, const void* scales_up,
                             const void* codebook_up, const uint32_t* codes_down, const void* scales_down,
                             const void* codebook_down, int pack_bits, int kc, int dim, int group, int64_t E,
                             int dtype, void* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The packed VQ experts of a SparseMoeBlock from its router logits, in one
 * call (qwen3_5.py:174-182 over the artifact's packed VQSwitchLinear
 * experts): the router of kmi_moe_route (inds [T, k] int32 and scores
 * [T, k] bf16 written, bit for bit as kmi_moe_route gives them), then
 * kmi_vq_packed_switch_glu with the weighted combine into out [T, H].
 * logits [T, E] bf16.  Up to 16 (token, slot) pairs with E <= 256 the
 * gate/up kernel routes each pair's token itself (no router launch);
 * otherwise it routes first, and up to 256 pairs over up to 256 experts
 * the expert-tile kernels form their tiles from the routed experts (no
 * sort launch).
 * k <= 8, E <= 1024.  workspace: kmi_vq_packed_switch_glu_workspace_bytes.
 */
int kmi_vq_packed_experts(const void* x, const void* logits, int64_t T, int64_t H, int64_t I, int k,
                          const uint32_t* codes_gate, const void* scales_gate, const void* codebook_gate,
                          const uint32_t* codes_up, const void* scales_up, const void* codebook_up,
                          const uint32_t* codes_down, const void* scales_down, const void* codebook_down,
                          int pack_bits, int kc, int dim, int group, int64_t E, int dtype, void* out,
                          int32_t* inds, void* scores, void* workspace, size_t workspace_bytes, void* stream);

int kmi_vq_switch_glu(const void* x, int64_t T, int64_t H, int64_t I, int k, const int32_t* inds,
                      const void* scores, const void* codes_gate, const void* scales_gate,
                      const void* codebook_gate, const void* codes_up, const void* scales_up,
                      const void* codebook_up, const void* codes_down, const void* scales_down,
                      const void* codebook_down, int code_bytes, int kc, int dim, int scale_group,
                      int64_t E, int dtype, void* out, void* workspace, size_t workspace_bytes,
                      void* stream);

/*
 * The VQ experts of a SparseMoeBlock from its router logits, in one call
 * (qwen3_5.py:174-182 over VQSwitchLinear experts): the router of
 * kmi_moe_route (inds [T, k] int32 and scores [T, k] bf16 written, bit for
 * bit as kmi_moe_route gives them), then kmi_vq_switch_glu with the
 * weighted combine into out [T, H].  logits [T, E] bf16.  For one token on
 * the MFMA path (per-channel scales, E <= 256) the gate/up kernel routes
 * the token itself, so the call is two kernel launches; otherwise it
 * routes first, and up to 256 pairs over up to 256 experts the expert
 * kernels form their tiles from the routed experts (no sort launch).
 * k <= 8, E <= 1024.  workspace:
 * kmi_vq_switch_glu_workspace_bytes(T, H, I, k).
 */
int kmi_vq_experts(const void* x, const void* logits, int64_t T, int64_t H, int64_t I, int k,
                   const void* codes_gate, const void* scales_gate, const void* codebook_gate,
                   const void* codes_up, const void* scales_up, const void* codebook_up,
                   const void* codes_down, const void* scales_down, const void* codebook_down, int code_bytes,
                   int kc, int dim, int scale_group, int64_t E, int dtype, void* out, int32_t* inds,
                   void* scores, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Calibration only (no counterpart in the reference): reads `bytes` of
 * device memory at `p` with `workgroups` workgroups of 16-byte nontemporal
 * loads, as the GEMV kernels load their weights, and computes nothing, so
 * a timed call gives the HBM read rate the GPU reaches at that size (the
 * measured ceiling beside the published 8 TB/s).  `out` (one uint32) is
 * written only for data whose XOR is a fixed value no test relies on.
 * bytes: a positive multiple of 16 under 2 GiB.
 */
int kmi_read_probe(const void* p, int64_t bytes, int workgroups, uint32_t* out, void* stream);

/*
 * Calibration only (no counterpart in the reference): `workgroups`
 * workgroups of 8 waves (two per SIMD, as the prefill GEMM runs) each issue
 * `iters` rounds of 16 v_mfma_f32_32x32x16_bf16 per wave into 2 x 2
 * accumulators on register operands (from the 64 uint32 at `seed`), so a
 * timed call gives the bf16 MFMA rate the GPU reaches (2 x 32 x 32 x 16
 * FLOPs per MFMA).  stamps (two uint64, device memory) receive workgroup
 * 0's first wave's shader-clock cycles and 100 MHz counter ticks around its
 * loop: their ratio is the clock under that load.  `out` (one uint32) is
 * written only for a sum no caller relies on.  iters: 1 .. 2^24.
 */
int kmi_mfma_probe(const uint32_t* seed, int workgroups, int iters, uint32_t* out, uint64_t* stamps,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KNURLOGIC_AMD_H */
