/*
 * ldk.h: C ABI of the MI355X (gfx950) decode hot-path library `libldk_amd.so`.
 *
 * Covers the W4A16 int4-weight matmul, the FP8 (OCP e4m3) weight-only matmul, fused
 * RMSNorm(+residual) and fused SwiGLU of Charlie-Gzz/llm-decode-kernels, plus the int4/fp8 weight
 * format routines. Each entry point names the reference interface it replaces (paths relative to
 * the reference repository).
 *
 * Conventions shared by every entry point:
 *  - All tensor pointers are DEVICE pointers owned by the caller. The library never allocates,
 *    frees, synchronizes or keeps a reference, so every call is safe inside hipGraph capture.
 *  - `stream` is a hipStream_t (passed as void*); 0 means the legacy default stream.
 *  - Matrices are row-major. `ld*` arguments are row strides in elements.
 *  - Activations, scales, zeros and outputs are fp16 unless a `dtype` argument says otherwise.
 *  - Return value: LDK_OK (0) or one of the LDK_ERR_* codes. On failure nothing is launched and
 *    ldk_last_error() returns a message for the calling thread.
 *  - Sizes are int64_t; every count must be > 0 unless stated.
 */
#ifndef LDK_H_
#define LDK_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LDK_ABI_VERSION 1

enum ldk_status {
  LDK_OK = 0,
  LDK_ERR_INVALID = 1,     /* bad argument: null pointer, size, shape or dtype */
  LDK_ERR_ALIGN = 2,       /* pointer or row stride not aligned as the kernel requires */
  LDK_ERR_UNSUPPORTED = 3, /* valid but not covered (e.g. M > 16 on the decode entry point) */
  LDK_ERR_LAUNCH = 4       /* the HIP runtime rejected the launch */
};

enum ldk_dtype { LDK_F16 = 0, LDK_BF16 = 1, LDK_F32 = 2 };

/* Flags for the matmul entry points (`flags`). Zero = let the library choose. */
enum ldk_flags {
  LDK_FACTORED = 1,  /* W4A16: s * sum x*(q - z) per group (w4a16.py:116-119, FACTORED): the
                        VALU kernel for M <= 2, and always the MFMA kernel */
  LDK_EXACT = 2,     /* W4A16: dequantize each weight to fp16 exactly as dequantize_ref first (the
                        VALU kernels, M <= 8; not with LDK_PATH_MFMA) */
  LDK_PATH_VALU = 4, /* force the wave64 VALU (dot2) skinny kernel */
  LDK_PATH_MFMA = 8, /* force the MFMA kernel (decode rows; prefill rows in 32-row blocks) */
  LDK_PATH_GEMM = 64, /* W4A16: force the prefill GEMM (128-row tiles over all of K, exact
                         dequantization on the matrix cores); the library's choice for many rows */
  /* W4A16 tuning: chunks of loads a wave keeps in flight per round (bits 4-5; 0 = table) */
  LDK_CPW_1 = 16,
  LDK_CPW_2 = 32,
  LDK_CPW_4 = 48,
  LDK_CPW_MASK = 48
};

/* ABI version (LDK_ABI_VERSION) the library was built with. */
int ldk_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* ldk_last_error(void);

/* ---------------------------------------------------------------------- int4 weight format */

/* Packs q [K, N] int32 (values 0..15) into packed [K/8, N] int32: nibble i of word [r, n] is
 * q[8r+i, n]. Replaces kernels/quant.py:20-28 (pack_int4). K % 8 == 0. */
int ldk_int4_pack(const int32_t* q, int32_t* packed, int64_t K, int64_t N, void* stream);

/* Inverse of ldk_int4_pack: packed [K/8, N] -> q [K, N] int32 in 0..15.
 * Replaces kernels/quant.py:31-35 (unpack_int4). */
int ldk_int4_unpack(const int32_t* packed, int32_t* q, int64_t K, int64_t N, void* stream);

/* Round-to-nearest asymmetric int4 quantization of w [N, K] (dtype LDK_F16/BF16/F32) with group
 * `group_size` along K: writes qweight [K/8, N] int32 and scales/zeros [K/group, N] in `dtype`.
 * Bit-identical to kernels/quant.py:38-49 (quantize_rtn). K % group_size == 0, group_size % 8 == 0. */
int ldk_quantize_rtn(const void* w, int dtype, int32_t* qweight, void* scales, void* zeros,
                     int64_t N, int64_t K, int group_size, void* stream);

/* Dequantizes to out [N, K] fp16 = (q - z) * s with one fp16 rounding, bit-identical to
 * kernels/reference.py:27-36 (dequantize_ref). group_size a power of two >= 8. */
int ldk_w4a16_dequant(const int32_t* qweight, const void* scales, const void* zeros, void* out,
                      int64_t N, int64_t K, int group_size, void* stream);

/* ------------------------------------------------------------------------------ W4A16 matmul */

/* Size of the split-K workspace the matmul entry points can use (bytes). The caller allocates
 * it once per device, zero-filled, 256-byte aligned, and passes it to every call. It holds one
 * 64-bit fixed-point accumulator per output of a split launch and, after them, one fp32 side
 * slot per output and split for partials outside the fixed-point range (|p| >= 2^21, inf, NaN);
 * the prefill GEMM's K split keeps fp32 partial tiles there. Every call leaves all of it zero
 * again, so it never needs re-clearing (also under graph replay). Calls that share one workspace
 * must be ordered (same stream or synchronized). */
int64_t ldk_workspace_bytes(void);

/* out [M, N] = x [M, K] @ dequant(qweight, scales, zeros)^T (+ bias [N]), fp32 accumulation,
 * fp16 output. Replaces kernels/w4a16.py:301-330 (w4a16_matmul) and its launch paths
 * w4a16.py:214-279. group_size a power of two in 32..256 dividing K; N % 4 == 0; x, qweight
 * 16-byte aligned with ldx % 8 == 0; scales, zeros 8-byte aligned. Prefill rows (M > 16) run
 * the prefill GEMM (group_size >= 64; 128-row tiles over all of K, every weight dequantized as
 * dequantize_ref does it, fp32 accumulation) or, for fewer rows, the MFMA kernel in 32-row blocks
 * without a cross-workgroup split (split_k is ignored there).
 *   block_n: output columns per workgroup, 16/32/64 (0 = table),
 *   split_k: workgroups splitting K per column tile (0 = table; > 1 needs the workspace),
 *   flags:   LDK_FACTORED / LDK_EXACT / LDK_PATH_VALU / LDK_PATH_MFMA, LDK_CPW_* (0 = table),
 *   workspace, workspace_bytes: the split-K workspace (NULL, 0: no cross-workgroup split). */
int ldk_w4a16_matmul(const void* x, int64_t ldx, const int32_t* qweight, const void* scales,
                     const void* zeros, const void* bias, void* out, int64_t ldo, int64_t M,
                     int64_t N, int64_t K, int group_size, int block_n, int split_k, int flags,
                     void* workspace, int64_t workspace_bytes, void* stream);

/* Decode-only entry (M <= 16; M > 16 returns LDK_ERR_UNSUPPORTED). Replaces the native
 * extension entry w4a16_decode of kernels/cuda/w4a16_decode.cu:136-181 and its wrapper
 * kernels/cuda/w4a16_cuda.py:45-56. split_k as in ldk_w4a16_matmul (0 = table). */
int ldk_w4a16_decode(const void* x, int64_t ldx, const int32_t* qweight, const void* scales,
                     const void* zeros, const void* bias, void* out, int64_t ldo, int64_t M,
                     int64_t N, int64_t K, int group_size, int split_k, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* Plan query: what ldk_w4a16_matmul runs for (M, N, K, group_size) with contiguous x and out
 * (ldx = K, ldo = N) and a workspace of ldk_workspace_bytes(). On entry *block_n, *split_k and
 * *flags are the tuning arguments a call would pass (all zero: the library's table); on return
 * they hold what runs: the output columns per workgroup, the workgroups splitting K per column
 * tile (the K splits of the prefill GEMM), and the path/mode/LDK_CPW_* flags (LDK_PATH_GEMM for
 * the prefill GEMM). Returns the status the call would return for those arguments, without
 * launching anything (a query needs no GPU). Replaces the choice tables of kernels/w4a16.py:282-298
 * (_pick_decode_path) and kernels/cuda/w4a16_cuda.py:29-42 (_pick_split), which are exported by
 * w4a16.py:333-355. */
int ldk_w4a16_config(int64_t M, int64_t N, int64_t K, int group_size, int* block_n,
                     int* split_k, int* flags);

/* Writes into buf (buf_len bytes, NUL-terminated) the name of the kernel instantiation that
 * ldk_w4a16_matmul runs for (M, N, K, group_size) with all-zero tuning arguments and a workspace
 * of ldk_workspace_bytes(), in the form the profiler lists it, e.g.
 * "w4a16_m1_kernel<8, 6, 4, 0, 1>". For reports that must name the kernel they measured. No
 * counterpart in the reference (its kernels are Triton programs named by their autotuner). */
int ldk_w4a16_kernel_name(int64_t M, int64_t N, int64_t K, int group_size, char* buf,
                          int64_t buf_len);

/* ldk_w4a16_matmul without a workspace argument, for callers that cannot allocate: code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc. No counterpart in the
 * reference. The split-K partial sums go to a library-owned device array of
 * LDK_NOALLOC_SCRATCH_BYTES per GPU (a file-scope __device__ array, held until the process ends);
 * the call allocates nothing. Its first call on a device looks up the array's device address and
 * clears it with one fill kernel on `stream`; the kernels leave it zero again after every call.
 * The plan is ldk_w4a16_matmul's with a workspace of that size (every default decode plan fits);
 * an explicit split_k whose partials do not fit returns LDK_ERR_INVALID with the bytes it needs.
 * All calls on one GPU share the array: calls that overlap on one GPU (unordered streams) race,
 * so order them (one stream, or events). Other arguments and results as ldk_w4a16_matmul. */
#define LDK_NOALLOC_SCRATCH_BYTES (4u << 20)
int ldk_w4a16_matmul_noalloc(const void* x, int64_t ldx, const int32_t* qweight,
                             const void* scales, const void* zeros, const void* bias, void* out,
                             int64_t ldo, int64_t M, int64_t N, int64_t K, int group_size,
                             int block_n, int split_k, int flags, void* stream);

/* Fused decode entries (M = 1, group_size 128). Each forms the activation row inside the W4A16
 * kernel's x staging instead of in a kernel of its own, one launch fewer per use. Same
 * qweight/scales/zeros/bias/out/workspace rules as ldk_w4a16_matmul.
 *
 * out [1, N] = rmsnorm(x (+ residual)) @ dequant(W)^T (+ bias) with x [K]: h = x (+ residual, fp16
 * add, written to residual_out); the activation is norm_weight * fp16(h * rsqrt(mean(h^2) + eps))
 * with the steps of ldk_rmsnorm. residual/residual_out both NULL or both set; residual_out must
 * not alias x or residual. Replaces the pair rmsnorm (kernels/rmsnorm.py:44-68) + w4a16_matmul
 * (kernels/w4a16.py:301-330) that the reference's OursBackend runs as norm then linear
 * (kernels/e2e/model.py:79-97). */
int ldk_w4a16_rmsnorm_matmul(const void* x, const void* residual, void* residual_out,
                             const void* norm_weight, float eps, const int32_t* qweight,
                             const void* scales, const void* zeros, const void* bias, void* out,
                             int64_t N, int64_t K, int group_size, void* workspace,
                             int64_t workspace_bytes, void* stream);

/* out [1, N] = swiglu(gate_up) @ dequant(W)^T (+ bias) with gate_up [2K] = [gate | up]: the
 * activation is fp16(silu(gate)) * up, bit-identical to ldk_swiglu. Replaces the pair
 * swiglu_fused (kernels/swiglu.py:56-61) + w4a16_matmul (kernels/w4a16.py:301-330) of the
 * reference's OursBackend act then linear (kernels/e2e/model.py:79-97). */
int ldk_w4a16_swiglu_matmul(const void* gate_up, const int32_t* qweight, const void* scales,
                            const void* zeros, const void* bias, void* out, int64_t N, int64_t K,
                            int group_size, void* workspace, int64_t workspace_bytes,
                            void* stream);

/* ----------------------------------------------------------------------------- FP8 (W8A16) */

/* Per-output-channel OCP e4m3 quantization of w [N, K] (dtype F16/BF16/F32): writes wq [K, N]
 * (e4m3fn bytes) and scale [N] in `dtype`. Bit-identical to kernels/fp8.py:25-30 (quantize_fp8). */
int ldk_fp8_quantize(const void* w, int dtype, uint8_t* wq, void* scale, int64_t N, int64_t K,
                     void* stream);

/* out [N, K] (scale's dtype, F16/BF16/F32) = e4m3(wq)^T * scale with one rounding.
 * Bit-identical to kernels/fp8.py:33-35 (dequantize_fp8). */
int ldk_fp8_dequant(const uint8_t* wq, const void* scale, int dtype, void* out, int64_t N,
                    int64_t K, void* stream);

/* out [M, N] = x [M, K] @ (e4m3(wq) * scale)^T (+ bias), fp32 accumulation, fp16 out.
 * wq [K, N] e4m3fn, scale [N] fp16. Replaces kernels/fp8.py:200-223 (w8a16_matmul) and its
 * kernels fp8.py:42-127, whose column masks take any N: here N % 4 == 0 (K % 8 == 0) and a
 * 16-byte aligned wq. block_n, split_k, flags and the workspace as for ldk_w4a16_matmul. More than
 * 64 rows run the prefill GEMM when N % 16 == 0 and K % 64 == 0, else the MFMA kernel in 16-row
 * blocks. */
int ldk_w8a16_matmul(const void* x, int64_t ldx, const uint8_t* wq, const void* scale,
                     const void* bias, void* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                     int block_n, int split_k, int flags, void* workspace, int64_t workspace_bytes,
                     void* stream);

/* Plan query for ldk_w8a16_matmul, as ldk_w4a16_config: *block_n, *split_k, *flags in = a
 * call's tuning arguments, out = what runs (columns per workgroup, K splits, LDK_PATH_VALU /
 * LDK_PATH_MFMA / LDK_PATH_GEMM) for contiguous x and out and a workspace of
 * ldk_workspace_bytes(); returns the status the call would return. Replaces the choice table of
 * kernels/fp8.py:175-187 (_pick), which the reference fills by timing. */
int ldk_w8a16_config(int64_t M, int64_t N, int64_t K, int* block_n, int* split_k, int* flags);

/* out [1, N] = (silu(g) * u) @ dequant_fp8(wq) (+ bias) for one row gate_up = [g | u] of 2K fp16
 * values: the activation is formed inside the W8A16 GEMV's x staging with the steps of
 * ldk_swiglu (bit-identical staged values), one launch instead of two. Same wq/scale/bias/
 * out/workspace rules as ldk_w8a16_matmul. Replaces the pair swiglu_fused (kernels/swiglu.py:56)
 * + w8a16_matmul (kernels/fp8.py:200) that the reference's OursFP8Backend runs as act then linear
 * (kernels/e2e/model.py:100-118). */
int ldk_w8a16_swiglu_matmul(const void* gate_up, const uint8_t* wq, const void* scale,
                            const void* bias, void* out, int64_t N, int64_t K, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* out [1, N] = rmsnorm(x (+ residual)) @ dequant_fp8(wq) (+ bias) for one row x [K]: the
 * activation norm_weight * fp16(h * rsqrt(mean(h^2) + eps)), h = x (+ residual, fp16 add, written
 * to residual_out), is formed inside the W8A16 GEMV's x staging with the steps of ldk_rmsnorm
 * (the row statistic is reduced in another order, so a staged value can differ from ldk_rmsnorm's
 * by one fp16 ulp). residual/residual_out both NULL or both set; residual_out must not alias x
 * or residual; x, norm_weight, residual, residual_out and wq 16-byte aligned. Replaces the pair
 * rmsnorm (kernels/rmsnorm.py:44-68) + w8a16_matmul (kernels/fp8.py:200) that the reference's
 * OursFP8Backend runs as norm then linear (kernels/e2e/model.py:79-118). */
int ldk_w8a16_rmsnorm_matmul(const void* x, const void* residual, void* residual_out,
                             const void* norm_weight, float eps, const uint8_t* wq,
                             const void* scale, const void* bias, void* out, int64_t N, int64_t K,
                             void* workspace, int64_t workspace_bytes, void* stream);

/* out [1, N] = x @ dequant_fp8(wq) (+ bias) with x [K] the decode attention output that
 * ldk_decode_attention_ranges left as partials (nq heads, max_len positions in ranges of rlen,
 * at *pos): each x value is the ranges' merge exp(m_r - max m)-weighted, o / l rounded once to
 * fp16, formed in the W8A16 GEMV's x staging with the arithmetic of
 * ldk_w4a16_attn_matmul_residual_stats's merge. K = nq * 128, at most 4 ranges
 * (ceil(max_len / rlen) <= 4), N % 4 == 0, pos 8-byte and wq 16-byte aligned; the pending
 * partials must be this stream's, max_len's, rlen's and nq's as for that entry (else
 * LDK_ERR_INVALID, no launch). One launch in place of the attention's merge launch and the FP8
 * o projection (the reference's attention block and FP8 linear, kernels/e2e/model.py:100-118,
 * 236-243). No counterpart entry exists in the reference. */
int ldk_w8a16_attn_matmul(const int64_t* pos, int64_t max_len, int64_t rlen, int nq, const uint8_t* wq,
                          const void* scale, const void* bias, void* out, int64_t N, int64_t K,
                          void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------- RMSNorm and SwiGLU */

/* Per row of x [M, N]: h = x (+ residual, fp16 add, written to res_out); out = weight * fp16(
 * h * rsqrt(mean(h^2) + eps)). residual/res_out both NULL or both set. Replaces
 * kernels/rmsnorm.py:44-68 (rmsnorm) and its kernel rmsnorm.py:15-37. */
int ldk_rmsnorm(const void* x, int64_t ldx, const void* residual, int64_t ldr, const void* weight,
                void* out, int64_t ldo, void* res_out, int64_t ldro, int64_t M, int64_t N,
                float eps, void* stream);

/* out [M, I] = fp16(silu(gate)) * up, silu in fp32. gate/up may be strided views of one fused
 * [M, 2I] tensor. Replaces kernels/swiglu.py:49-61 (swiglu, swiglu_fused) and its kernel
 * swiglu.py:14-28. */
int ldk_swiglu(const void* gate, int64_t ldg, const void* up, int64_t ldu, void* out, int64_t ldo,
               int64_t M, int64_t I, void* stream);

/* ------------------------------------------------------------------------ decode attention */

/* One decode step's attention block for one new token (batch 1) of one layer: RoPE on q and the
 * new k (cos/sin of *pos * inv_freq[i], rotate_half pairing, the reference's fp16 rounding
 * steps), the new k and v written at *pos into the static cache, then grouped-query softmax
 * attention of each of the nq heads over positions 0..*pos, in one launch.
 *   qkv:      [nq*head_dim + 2*nkv*head_dim] fp16, the qkv projection output (bias added);
 *   pos:      int64 device scalar, the new token's position (< max_len);
 *   inv_freq: [head_dim/2] fp32 RoPE inverse frequencies;
 *   k_cache:  fp16 K tiles, per kv head [max_len/32][2][4][16][32]: chunk c, row half hb, dim
 *             step s, row i, column e hold K[32c + 8(i/4) + 4hb + i%4][32s + e];
 *   vt_cache: fp16 V^T tiles, per kv head [max_len/32][8][16][32]: step t, dim block b, row r,
 *             column e hold V[32t + e][16b + r];
 *   out:      [nq*head_dim] fp16; scale: the softmax scale (head_dim^-0.5).
 * head_dim == 128, nq % nkv == 0, max_len a multiple of 32 (k_cache and vt_cache 16-byte
 * aligned). A *pos >= max_len writes nothing and attends over the whole cache; a negative *pos
 * writes nothing and returns zeros. Caches of more than 512 positions are split into up to 32
 * position ranges whose partials go through library-owned device memory to a second launch on
 * the same stream that merges them (graph capture is safe); calls on one device must be
 * stream-ordered. warm, warm_bytes, nwarm: byte ranges the launch reads into the caches for the
 * launches after it, as ldk_decode_attention_ranges takes them (nwarm = 0: none).
 * Replaces the per-layer attention of the
 * reference's runner for decode steps (kernels/e2e/model.py:212-243: RoPE, k/v index_copy_ into
 * the cache, scaled_dot_product_attention with the causal mask; the reference's cache is
 * [batch][kv][max_len][head_dim] for both K and V). */
int ldk_decode_attention(const void* qkv, const int64_t* pos, const float* inv_freq, void* k_cache,
                         void* vt_cache, void* out, int nq, int nkv, int head_dim, int64_t max_len,
                         float scale, const void* const* warm, const int64_t* warm_bytes, int nwarm,
                         void* stream);

/* ldk_decode_attention's range kernel alone, for a consumer that merges the ranges itself
 * (ldk_w4a16_attn_matmul_residual_stats): the cache is split into ranges of rlen positions (a
 * multiple of 32, at most 32 ranges), every range live at *pos (a lone one too) leaves its
 * {max, sum} and unnormalised output in library-owned device memory, and there is no merge
 * launch and no output. Cache write, numerics and argument rules as ldk_decode_attention;
 * nq <= 128. The partials stay valid until the next attention call on the device; calls must be
 * stream-ordered. The same launch can warm the caches for the launches after it: nwarm (0..8)
 * device ranges warm[k] of warm_bytes[k] bytes (16-byte aligned, multiples of 16, under 32 GiB
 * in all) are read by extra workgroups dispatched after the attention's, into the MALL and the
 * reading XCD's L2, while the attention's few workgroups leave the CUs idle; they change no
 * result and write nothing. No counterpart entry exists in the reference: it is one half of this
 * build's fusion of the attention's merge into the o projection (kernels/e2e/model.py:212-233
 * there). */
int ldk_decode_attention_ranges(const void* qkv, const int64_t* pos, const float* inv_freq, void* k_cache,
                                void* vt_cache, int nq, int nkv, int head_dim, int64_t max_len, int64_t rlen,
                                float scale, const void* const* warm, const int64_t* warm_bytes, int nwarm,
                                void* stream);

/* Prompt attention: T tokens of one sequence at positions pos[T] (int64 device array), in two
 * launches on `stream`: RoPE on q and k (the fp16 steps of ldk_decode_attention), the roped q
 * written to q_scratch [T][nq][128] fp16 (a caller-provided 16-byte aligned device buffer of
 * T * nq * 128 halves), k and v written into the tiled caches at every pos[t] in [0, max_len)
 * (others write nothing), then causal grouped-query softmax attention of each token t over the
 * cache positions 0..pos[t] (the cache then holds all T tokens; a negative pos[t] gives zeros).
 * qkv [T] rows of ldqkv >= (nq + 2 nkv) * 128 fp16 (projection output, bias added); out [T] rows
 * of ldo >= nq * 128 fp16. Cache layout, head_dim (128), nq % nkv and max_len rules as
 * ldk_decode_attention. Replaces the prompt branch of the reference runner's attention
 * (kernels/e2e/model.py:212-243: RoPE, k/v index_copy_ into the cache, scaled_dot_product_attention
 * with the causal mask), which is about twenty small launches per layer. */
int ldk_prefill_attention(const void* qkv, int64_t ldqkv, const int64_t* pos, int64_t T,
                          const float* inv_freq, void* k_cache, void* vt_cache, void* q_scratch,
                          void* out, int64_t ldo, int nq, int nkv, int head_dim, int64_t max_len,
                          float scale, void* stream);

/* Residual + RMSNorm carried across the two projections around it (decode, one row), as a pair
 * of launches that replaces linear + rmsnorm(x, residual) + linear of the reference's layer
 * (kernels/e2e/model.py:79-97, 226-233: o_proj, post_attention_layernorm, gate_up). Group size
 * 128. No counterpart entry exists in the reference; it is this build's fusion of its pair.
 *
 * ldk_w4a16_matmul_residual_stats: h_out [N] = fp16(fp16(x @ dequant(W)^T (+ bias)) + residual)
 * (the linear's fp16 output, then the norm's fp16 residual add) and row_stats[t] = the sum of
 * h^2 over column tile t, for ldk_w4a16_row_stats_count(N, K, group_size) tiles (at most 256).
 * h_out may alias residual (an in-place residual update), not x; residual and h_out 8-byte
 * aligned. ldk_w4a16_rmsnorm_stats_matmul: out [N] = rmsnorm(h) @ dequant(W)^T (+ bias) with the
 * statistic summed from those nstats partials; the activation norm_weight * fp16(h * rsqrt(
 * mean(h^2) + eps)) as ldk_rmsnorm forms it (the statistic's order differs, so a staged value can
 * differ from ldk_rmsnorm's by one fp16 ulp). norm_weight 16-byte aligned. */
int64_t ldk_w4a16_row_stats_count(int64_t N, int64_t K, int group_size); /* < 0: -ldk_status */
int ldk_w4a16_matmul_residual_stats(const void* x, const void* residual, void* h_out, float* row_stats,
                                    const int32_t* qweight, const void* scales, const void* zeros,
                                    const void* bias, int64_t N, int64_t K, int group_size,
                                    void* workspace, int64_t workspace_bytes, void* stream);
/* ldk_w4a16_matmul_residual_stats with x the attention output that ldk_decode_attention_ranges
 * left as partials (nq heads, max_len positions in ranges of rlen, at *pos): each x value is the
 * ranges' merge exp(m_r - max m)-weighted, o / l rounded once to fp16, formed in the projection's
 * x staging (the merge launch's arithmetic; the sum of the weighted l is a chain in range order
 * there, a lane reduction in the merge launch, so x can differ from it in the last fp16 bit).
 * K = nq * 128, at most 4 ranges (ceil(max_len / rlen) <= 4), group size 128, pos 8-byte aligned.
 * The last ldk_decode_attention_ranges call on the device must have left its partials on this
 * stream with this max_len, rlen and nq, and no ldk_decode_attention range launch (a cache of
 * more than 512 positions) may have overwritten them since: else LDK_ERR_INVALID, no launch.
 * One launch in place of the attention's merge launch and the projection. No counterpart entry
 * exists in the reference. */
int ldk_w4a16_attn_matmul_residual_stats(const int64_t* pos, int64_t max_len, int64_t rlen, int nq,
                                         const void* residual, void* h_out, float* row_stats,
                                         const int32_t* qweight, const void* scales, const void* zeros,
                                         const void* bias, int64_t N, int64_t K, int group_size,
                                         void* workspace, int64_t workspace_bytes, void* stream);
int ldk_w4a16_rmsnorm_stats_matmul(const void* h, const float* row_stats, int nstats,
                                   const void* norm_weight, float eps, const int32_t* qweight,
                                   const void* scales, const void* zeros, const void* bias,
                                   void* out, int64_t N, int64_t K, int group_size,
                                   void* workspace, int64_t workspace_bytes, void* stream);

/* Prefill rows of a gate_up projection with SwiGLU in the prefill GEMM's epilogue. No counterpart
 * entry exists in the reference, whose runner runs the activation as a kernel of its own
 * (kernels/e2e/model.py:79-97, kernels/swiglu.py:49-61). out [M, N/2] (row stride ldo >= N/2,
 * ldo % 4 == 0, 8-byte aligned) = swiglu_fused(x @ dequant(W)^T (+ bias)) with g the product's
 * columns [0, N/2) and u [N/2, N): the standalone SwiGLU's steps on the fp16 products, so bit for
 * bit ldk_w4a16_matmul then ldk_swiglu. Only where ldk_w4a16_matmul_swiglu_applies(M, N, K,
 * group_size) returns 1 (the library's plan for the shape is the prefill GEMM on tiles of at most
 * 64 rows with an even number of column groups and no K split); else LDK_ERR_UNSUPPORTED and no
 * launch. */
int ldk_w4a16_matmul_swiglu_applies(int64_t M, int64_t N, int64_t K, int group_size);
int ldk_w4a16_matmul_swiglu(const void* x, int64_t ldx, const int32_t* qweight, const void* scales,
                            const void* zeros, const void* bias, void* out, int64_t ldo, int64_t M, int64_t N,
                            int64_t K, int group_size, void* workspace, int64_t workspace_bytes, void* stream);

/* The e4m3 twin (weights wq [K, N] e4m3 with the per-column scale, as ldk_w8a16_matmul): out
 * [M, N/2] = swiglu_fused(x @ (wq * scale) (+ bias)), bit for bit ldk_w8a16_matmul then
 * ldk_swiglu; no counterpart entry in the reference (its FP8 runner runs the activation as a
 * kernel of its own, kernels/e2e/model.py:100-118). Only where ldk_w8a16_matmul_swiglu_applies
 * returns 1 (as above, on 4-wave tiles only: gate_up 17920x1536 from 200 to 512 rows); else
 * LDK_ERR_UNSUPPORTED and no launch. */
int ldk_w8a16_matmul_swiglu_applies(int64_t M, int64_t N, int64_t K);
int ldk_w8a16_matmul_swiglu(const void* x, int64_t ldx, const uint8_t* wq, const void* scale, const void* bias,
                            void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------- greedy decode bookkeeping */

/* idx = argmax(logits[0:V]) (torch.argmax order: NaN largest, lowest index on ties), then
 * out[*pos] = idx when 0 <= *pos < out_len (out may be NULL), *tok = idx, *pos += 1; one launch,
 * no memset. Its workgroups meet in library-owned device state that the launch leaves zeroed,
 * so it replays safely inside a hipGraph; calls on one device must be stream-ordered. logits dtype
 * LDK_F16/BF16/F32; tok, out and pos are int64 device pointers. Replaces the greedy step of
 * kernels/e2e/run.py:69-74 (argmax, out.index_copy_, tok.copy_, pos.add_). */
int ldk_greedy_step(const void* logits, int dtype, int64_t V, int64_t* tok, int64_t* out,
                    int64_t out_len, int64_t* pos, void* stream);

/* ------------------------------------------------------------------ fp16 lm_head (one row) */

/* y[n] = fp16(sum_k w[n*ldw + k] * x[k]) for n < N: the tied fp16 lm_head of the decode step,
 * `F.linear(h, self.lm_head)` at one row (kernels/e2e/model.py:253). x fp16 [K], w fp16 [N, ldw]
 * row-major, y fp16 [N]; fp32 accumulation, one rounding. K and ldw multiples of 8, K <= 2048,
 * x and w 16-byte aligned. rows_per_wave: 0 (library choice), 4 or 8. */
int ldk_f16_gemv(const void* x, const void* w, int64_t ldw, void* y, int64_t N, int64_t K,
                 int rows_per_wave, void* stream);

/* ldk_f16_gemv on x = rmsnorm(h (+ residual)) * norm_weight, formed in the kernel's x staging:
 * the final `self.norm(h, residual)` and the head of kernels/e2e/model.py:250-253 in one launch
 * (the norm's steps are rmsnorm_ref's, kernels/reference.py:9-19; h + residual is not written
 * back). residual may be NULL; h, residual and norm_weight are fp16 [K], 16-byte aligned. */
int ldk_f16_rmsnorm_gemv(const void* h, const void* residual, const void* norm_weight, float eps,
                         const void* w, int64_t ldw, void* y, int64_t N, int64_t K,
                         int rows_per_wave, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LDK_H_ */
