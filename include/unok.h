/*
 * unok.h -- C-ABI of the uno_amd kernel library (libunok.so, gfx950 / MI355X).
 *
 * The drop-in boundary for Uno's conditional-LoRA block-diffusion training step. The reference
 * (ifm-ai/uno) has no native code: every hot op of its step runs in library kernels reached from
 * Python. Each entry point below replaces one of those call sites; the citation after each
 * declaration names the reference code (file:line) whose semantics it implements.
 *
 * Conventions
 *   - Return 0 on success, a positive hipError_t for a failed launch, or a negative code for an
 *     argument error (-1 invalid value, -2 alignment, -3 unsupported); unok_last_error() returns
 *     the message of the calling thread's last failure.
 *   - Tensors are device pointers with explicit row strides in ELEMENTS (unless named *_bytes);
 *     dtype codes: 0 = float32, 1 = bfloat16. The caller owns all memory; no entry point
 *     allocates or frees device memory. All work is enqueued on `stream` (a hipStream_t).
 *   - Attention masks are per-row key intervals: int32[8] per row =
 *     {lo1, hi1, lo2, hi2, qlo2, qhi2, 0, segment_length}; source 1 = clean-stream K/V,
 *     source 2 = noisy-stream K/V; [qlo2, qhi2) = source-2 query rows that see this key row.
 */
#ifndef UNOK_H
#define UNOK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int unok_abi_version(void);
const char* unok_last_error(void);

/* ---- Linear layers with the token-gated LoRA update fused in ---------------------------- */

/* C = alpha * gate (.) (A[M,K] B[N,K]^T + A2[:, seg_col(n) : +K2] B2[N,K2]^T) + R.
 * Forward of a LoRA linear: A = x, B = W, A2 = h = m (.) (x A_lora^T), B2 = (alpha/r) B_lora.
 * Data gradient: A = dY, B = W^T (resident transposed copy), A2 = g, B2 = A_lora^T.
 * Replaces: PEFT lora.Linear.forward (peft 0.15.2) with the token gate of
 * training/lora.py:164-174 and the frozen base F.linear of the Qwen3 projections
 * (transformers/models/qwen3/modeling_qwen3.py:81-82,241-253); LM head of
 * training/losses.py:30 and training/trainer.py:238-247. */
int unok_gemm_nt(int in_dtype, int out_dtype, int M, int N, int K,
                 const void* A, int64_t lda, const void* B, int64_t ldb,
                 const void* A2, int64_t lda2, const void* B2, int64_t ldb2, int K2,
                 int nseg, const int* seg_end, const int* seg_col,
                 void* C, int64_t ldc, const void* R, int64_t ldr,
                 const uint8_t* gate, float alpha, void* stream);

/* C[M, N/2] = silu(G) (.) U of the gate/up product A[M,K] B[N,K]^T (+ A2[M,K2] B2[N,K2]^T, the
 * LoRA extension), bf16, for B (and B2) with 64-row interleaved gate/up rows (rows 128 b + [0, 64):
 * gate features 64 b + [0, 64); rows 128 b + [64, 128): the same up features); rounded exactly as
 * unok_gemm_nt followed by unok_swiglu_fwd. With gu non-null, also stores the product itself as
 * gu[M, N] = [gate | up] (the layout of the plain product, for the backward). M and N multiples of
 * 256, K of 64 and K2 of 32; A2 may be null (K2 ignored). The remote Qwen3 decoder's MLP input to
 * down_proj, act_fn(gate_proj(x)) * up_proj(x) (modeling_qwen3.py:81-82), with the LoRA terms of
 * gate_proj and up_proj (peft 0.15.2 lora.Linear; training/lora.py:136-179). */
int unok_gemm_nt_swiglu(int M, int N, int K, const void* A, int64_t lda, const void* B, int64_t ldb,
                        const void* A2, int64_t lda2, const void* B2, int64_t ldb2, int K2,
                        void* C, int64_t ldc, void* gu, int64_t ldgu, void* stream);

/* dgu[M, 2F] = SwiGLU backward of dS = A[M,K] B[F,K]^T + A2[M,K2] B2[F,K2]^T against
 * gu[M, 2F] = [gate | up] (dS is never stored); bf16, rounded exactly as unok_gemm_nt followed by
 * unok_swiglu_bwd. M and F multiples of 256, K of 64, K2 of 32. Backward of the remote decoder's MLP
 * act_fn(gate_proj(x)) * up_proj(x) through down_proj (modeling_qwen3.py:81-82) with the LoRA
 * data-gradient extension of down_proj (peft 0.15.2 lora.Linear). */
int unok_gemm_nt_swiglu_bwd(int M, int F, int K, const void* A, int64_t lda, const void* B, int64_t ldb,
                            const void* A2, int64_t lda2, const void* B2, int64_t ldb2, int K2,
                            const void* gu, int64_t ldgu, void* dgu, int64_t lddgu, void* stream);

/* Gated LoRA linear for decode and draft blocks (bf16), where M = sequences x block rows (128 for 8
 * sequences of 16) and the product streams the weight once:
 *   y = A B^T + H[:, seg_col(n) : +r] LB[n, :r]^T + Res,  H = bf16(gate (.) (A LA^T))  [M, R],
 * A [M,K] activations, B [N,K] weight, LA [R,K] the LoRA A rows of all segments, LB [N,r] the
 * (alpha/r)-scaled LoRA B; segment i covers output columns [seg_end[i-1], seg_end[i]) and reads
 * H columns [seg_col[i], seg_col[i] + r). LA null: no LoRA (R, LB, r and the segments ignored).
 * epilogue 0: C[M,N] = y;  epilogue 1: C[M,N/2] = silu(G) (.) U of y = [G | U] (no Res), rounded as
 * y in bf16 followed by unok_swiglu_fwd. The product runs on 128 x 128 output tiles (the LA rows are
 * extra columns), each split into `splits` ranges of the K tiles (splits <= 0: chosen from the
 * shape) so the grid fills the chip; the ranges' fp32 partial sums go through `workspace` (at
 * least unok_gemm_nt_rows_workspace() bytes, 16-byte aligned) and a second kernel adds them in
 * range order (the result does not depend on timing), forms H and applies the rank-r update and
 * the epilogue. One range without LoRA and epilogue 0 writes C directly and needs no workspace.
 * K a multiple of 128, N of 4 (of 32 for epilogue 1), R and r of 8 (R at most 512, r at most 128),
 * segment ends (but the last) of 16 and segment columns of 8.
 * Replaces: the LoRA linear of the draft forward, nano_vllm_uno/layers/linear.py:241-307 (base
 * projection plus lora_B(lora_A(x) * lora_mask) * scaling, the mask off on the seed row), called
 * from engine/two_pass_decoding.py:273-283, and the MLP activation that follows gate_up_proj
 * (SiluAndMul, nano_vllm_uno/layers/activation.py:6, applied at nano_vllm_uno/models/qwen3.py:128-132). */
int64_t unok_gemm_nt_rows_workspace(int M, int N, int K, int R, int epilogue, int splits);
int unok_gemm_nt_rows(int M, int N, int K, const void* A, int64_t lda, const void* B, int64_t ldb,
                      const void* LA, int64_t ldla, int R, const void* LB, int64_t ldlb, int r,
                      int nseg, const int* seg_end, const int* seg_col,
                      void* C, int64_t ldc, const void* Res, int64_t ldres, const uint8_t* gate,
                      int epilogue, int splits, void* workspace, int64_t ws_bytes, void* stream);

/* C[P,Q] (fp32) = beta * C + alpha * A[Mrows,P]^T B[Mrows,Q] (split-K over rows through a
 * caller workspace of unok_gemm_tn_workspace() bytes). LoRA weight gradients
 * dB = s dY^T h, dA = g^T x. Replaces: autograd of lora_A / lora_B (peft 0.15.2) under
 * training/lora.py:83-91 (fp32 adapter weights). */
int64_t unok_gemm_tn_workspace(int Mrows, int P, int Q);
int unok_gemm_tn(int in_dtype, int Mrows, int P, int Q, const void* A, int64_t lda,
                 const void* B, int64_t ldb, float* C, int64_t ldc, float alpha, float beta,
                 void* workspace, int64_t ws_bytes, void* stream);

/* unok_gemm_tn without a workspace argument and without any device allocation: the split-K
 * partials live in a 64 MiB array the library holds on each GPU it runs on (resolved on the first
 * call on that device; the stream must belong to the current device). No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Problems whose partials exceed 64 MiB
 * (unok_gemm_tn_workspace(Mrows, P, Q) > 67108864) are rejected with -1. All calls on one GPU
 * share the array: calls that overlap on that GPU race. */
int unok_gemm_tn_noalloc(int in_dtype, int Mrows, int P, int Q, const void* A, int64_t lda,
                         const void* B, int64_t ldb, float* C, int64_t ldc, float alpha, float beta,
                         void* stream);

/* ---- Row-wise decoder ops ----------------------------------------------------------------- */

/* y = round(x * rsqrt(mean(x^2) + eps) * w) (one rounding), rstd[M] saved. Qwen3RMSNorm
 * (modeling_qwen3.py:50-64); input/post-attention/final norms of the remote decoder. */
int unok_rmsnorm_fwd(int dtype, int M, int H, const void* x, int64_t ldx, const void* w,
                     void* y, int64_t ldy, float* rstd, float eps, void* stream);
/* dx = rstd (g - xhat mean(g xhat)) + dres, g = dy * w. dx may alias dres. */
int unok_rmsnorm_bwd(int dtype, int M, int H, const void* dy, const void* x, const void* w,
                     const float* rstd, const void* dres, void* dx, void* stream);

/* Per-head q/k RMSNorm (wq/wk may both be null: RoPE only) then rotate_half RoPE with
 * angle fl32(pos * inv_freq[i]), in fp32 with one rounding at the store; writes contiguous
 * q [M, nq*d] and k [M, nk*d], and, when v_out is non-null, the v heads of qkv into v_out
 * [M, nk*d] (row stride ldv). dtype: q, k, v_out and the weights; qkv_dtype: the qkv input
 * (dtype, or fp32 with bf16 outputs).
 * modeling_qwen3.py:140-160 (rotary), :237-253 (q_norm/k_norm before RoPE). */
int unok_qknorm_rope_fwd(int dtype, int qkv_dtype, int M, int nq, int nk, int d, const void* qkv,
                         int64_t ld, const void* wq, const void* wk, const int64_t* pos,
                         const float* inv_freq, float eps, void* q_out, void* k_out, void* v_out,
                         int64_t ldv, float* rstd, void* stream);
/* dtype: dqkv and the weights; grad_dtype: dq and dk (dtype, or fp32 with a bf16 dqkv); x_dtype:
 * the pre-norm q/k columns read from qkv (row stride ld): grad_dtype, or bf16 beside fp32 gradients. */
int unok_qknorm_rope_bwd(int dtype, int grad_dtype, int x_dtype, int M, int nq, int nk, int d,
                         const void* dq, const void* dk, const void* qkv, int64_t ld, const void* wq,
                         const void* wk, const int64_t* pos, const float* inv_freq,
                         const float* rstd, void* dqkv, int64_t ldd, void* stream);
/* cos_tab / sin_tab [P, half] = cos / sin of fl32(p * inv_freq[j]): the RoPE angles of the fused
 * q|k|v projection epilogue (modeling_qwen3.py:140-160). */
int unok_rope_table(int P, int half, const float* inv_freq, float* cos_tab, float* sin_tab, void* stream);

/* q|k|v projection (+ LoRA extension) with the q/k RMSNorm and RoPE in the GEMM epilogue, bf16, head
 * dim 128: the product stays fp32 until each q/k head is normalised (wq / wk, or both null), scaled
 * and rotated, then q [M, 128 nq], k and v [M, 128 nk] are stored in bf16; rstd [M, nq+nk] and the
 * pre-norm q/k columns in bf16, qk_pre [M, 128 (nq+nk)], when non-null. Replaces the q/k/v
 * projections of the remote Qwen3 attention with their gated LoRA (modeling_qwen3.py:237-253,
 * training/lora.py:164-174). M and 128 (nq + 2 nk) multiples of 256, K of 64, K2 of 32. */
int unok_gemm_nt_qkv_rope(int M, int K, int nq, int nk, const void* A, int64_t lda, const void* B,
                          int64_t ldb, const void* A2, int64_t lda2, const void* B2, int64_t ldb2, int K2,
                          int nseg, const int* seg_end, const int* seg_col, const void* wq, const void* wk,
                          const int64_t* pos, const float* cos_tab, const float* sin_tab, int P, float eps,
                          void* q_out, void* k_out, void* v_out, float* rstd, void* qk_pre, void* stream);

/* out = silu(gate) * up over the fused [gate | up] projection, rounded once (modeling_qwen3.py:81-82). */
int unok_swiglu_fwd(int dtype, int M, int F, const void* gu, int64_t ld, void* out, void* stream);
int unok_swiglu_bwd(int dtype, int M, int F, const void* dout, const void* gu, int64_t ld,
                    void* dgu, int64_t ldd, void* stream);

/* Embedding lookup (remote Qwen3 embed_tokens) and index-mapped row copies (the region
 * split of training/modeling.py:101-113 and the [noisy|clean] layout of :65-81). */
int unok_embedding(int elem_bytes, int M, int H, const int64_t* ids, const void* table,
                   int64_t vocab, void* out, void* stream);
int unok_rows_copy(int row_bytes, int M, const void* src, int64_t ld_src_bytes,
                   const int32_t* smap, void* dst, int64_t ld_dst_bytes,
                   const int32_t* dmap, void* stream);

/* ---- Block-diffusion attention ------------------------------------------------------------- */

/* O = softmax(Q K^T / sqrt(d) over the row's key intervals) V with GQA (q head h -> kv head
 * h / (Hq/Hkv)); LSE[Mq,Hq] = log2-sum-exp2 of the scaled scores. Replaces torch flex_attention
 * with the BlockMask of the remote prepare_for_bd_training (training/train.py:142,
 * training/trainer.py:198-218). */
int unok_attn_fwd(int dtype, int Mq, int Hq, int Hkv, int D, const void* Q, int64_t ldq,
                  const void* K1, int64_t ldk1, const void* V1, int64_t ldv1,
                  const void* K2, int64_t ldk2, const void* V2, int64_t ldv2,
                  const int32_t* iv, void* O, int64_t ldo, float* LSE, float scale,
                  void* stream);
/* dQ for every query; dK/dV for the source-2 keys when dK/dV are non-null (source-1 keys are
 * the detached clean stream). Dsum [Mq,Hq] fp32 is caller scratch. grad_dtype: dQ and dK (dtype,
 * or fp32 with bf16 inputs); dV has dtype. */
int unok_attn_bwd(int dtype, int grad_dtype, int Mq, int Mk2, int Hq, int Hkv, int D, const void* Q,
                  int64_t ldq,
                  const void* K1, int64_t ldk1, const void* V1, int64_t ldv1,
                  const void* K2, int64_t ldk2, const void* V2, int64_t ldv2,
                  const int32_t* iv, const int32_t* ivk, const void* O, int64_t ldo,
                  const float* LSE, const void* dO, int64_t lddo, float* Dsum,
                  void* dQ, int64_t lddq, void* dK, int64_t lddk, void* dV, int64_t lddv,
                  float scale, void* stream);

/* The noisy stream's backward with the q/k RMSNorm + RoPE backward (modeling_qwen3.py:140-160,
 * 237-253) applied to the fp32 dQ / dK accumulators: dqkv [Mq, (Hq + 2 Hkv) D] receives the
 * gradient before the norm in its q and k column blocks and dV in its v block (bf16; source-2
 * keys are the query rows, Mk2 = Mq). pre [Mq, (Hq + Hkv) D] = the pre-norm q/k columns (bf16),
 * rstd [Mq, Hq + Hkv] their 1/rms, cos_tab / sin_tab [P, D/2] the angles (unok_rope_table) at
 * each row's position; wq / wk null: RoPE only. Dsum [Mq, Hq] fp32 is caller scratch. */
int unok_attn_bwd_qknorm(int Mq, int Hq, int Hkv, int D, const void* Q, int64_t ldq, const void* K1,
                         int64_t ldk1, const void* V1, int64_t ldv1, const void* K2, int64_t ldk2,
                         const void* V2, int64_t ldv2, const int32_t* iv, const void* O, int64_t ldo,
                         const float* LSE, const void* dO, int64_t lddo, float* Dsum, const void* pre,
                         int64_t ldpre, const float* rstd, const void* wq, const void* wk,
                         const int64_t* pos, const float* cos_tab, const float* sin_tab, int P,
                         void* dqkv, int64_t lddqkv, float scale, void* stream);

/* ---- Draft-block attention over the KV cache -------------------------------------------------- */

/* q/k RMSNorm + RoPE of a draft block's fused qkv rows [B*L, (nq + 2 nk) * D] (the arithmetic of
 * unok_qknorm_rope_fwd; wq / wk null: no q/k norm), at positions lengths[b] + t; the block's K and V
 * rows into this layer's caches kc / vc [B, nk, max_len, D] at rows lengths[b] + t (rows at or past
 * max_len are not written); the queries into qd [B * nk * 128, D]: the rep = nq / nk q heads of
 * K/V head kv and sequence b fill rows 128 (b nk + kv) + L (h % rep) + t, the other rows of each
 * 128 are zeroed. bf16, D in {64, 128}, rep * L <= 128. Replaces: the q/k norm and rotary embedding
 * of Qwen3Attention.forward (nano_vllm_uno/models/qwen3.py:81-99) and the KV-cache store of
 * nano_vllm_uno/layers/attention.py:628-668 (BLOCK_DECODE). */
int unok_decode_prep(int B, int L, int nq, int nk, int D, const void* qkv, int64_t ld, const void* wq,
                     const void* wk, const int64_t* lengths, const float* inv_freq, float eps, void* kc,
                     void* vc, int max_len, void* qd, void* stream);
/* Split-key attention of draft blocks: S * QR rows, row i attending with query Q[i % QR] (one
 * head) to K / V rows over its interval iv[i] (int32[8], keys [iv[0], iv[1])), O and LSE per row
 * as unok_attn_fwd. The S rows of one query cover disjoint ranges of its cache keys, so the grid
 * holds S workgroups per (sequence, K/V head) pair. Replaces: the causal flash attention over the
 * cache of nano_vllm_uno/layers/attention.py:658-666 (flash_attn_with_kvcache, causal=True). */
int unok_attn_fwd_split(int QR, int S, int D, const void* Q, int64_t ldq, const void* K, int64_t ldk,
                        const void* V, int64_t ldv, const int32_t* iv, void* O, int64_t ldo, float* LSE,
                        float scale, void* stream);
/* out[dst[i]] (rows of D) = merge of the S partial rows s * QR + i of unok_attn_fwd_split by their
 * log-sum-exp weights (rows with dst[i] < 0 are skipped). The split-key combine inside the flash
 * attention that nano_vllm_uno/layers/attention.py:658-666 calls. */
int unok_attn_split_combine(int QR, int S, int D, const void* opart, int64_t ldp, const float* lse,
                            const int32_t* dst, void* out, int64_t ldo, void* stream);

/* ---- Block-diffusion batch preparation ----------------------------------------------------- */

/* Noising, [noisy | clean] concatenation, stream maps and interval tables of one batch.
 * The model-side contract of prepare_for_bd_training (call site training/trainer.py:198-209;
 * region layout training/modeling.py:65-81; uniform replacement range [1, mask_id) of
 * nano_vllm_uno/engine/noise.py:24-26). */
int unok_bd_prepare(int B, int L, const int64_t* ids, const int64_t* pos, const uint8_t* prompt,
                    int block_size, int mask_id, int noise_mask_mode, int intra_causal,
                    uint64_t key, int64_t* concat_ids, int64_t* concat_pos, uint8_t* region,
                    uint8_t* noised, float* tfull, int32_t* noisy_src, int32_t* clean_src,
                    int32_t* noisy_iv, int32_t* clean_iv, int64_t* noisy_ids,
                    int64_t* clean_ids, void* stream);
/* region[B, 2L] = the [noisy | clean] per-segment layout mask alone (1 on noisy rows), from the
 * model positions: segments start at t = 0 and wherever pos[t-1] >= pos[t]. Replaces
 * calculate_token_nums + _build_noisy_region_mask of prepare_uno_layout
 * (training/modeling.py:65-81,84-98). */
int unok_bd_region(int B, int L, const int64_t* pos, uint8_t* region, void* stream);
/* p_mask = noise level of every noised token in row-major order (training/trainer.py:278);
 * count[0] = their number and, when pos [n] is non-null, count[1] = the largest position (clamped to
 * [0, 2^31 - 1]), which sizes the RoPE tables. */
int unok_bd_compact(int64_t n, const uint8_t* noised, const float* tfull, const int64_t* pos,
                    float* p_mask, int32_t* count, void* stream);

/* ---- Objectives ------------------------------------------------------------------------------ */

/* Chunked LM-head cross-entropy with 1/t row weights (training/trainer.py:267-283): per vocab
 * chunk, merge running (max, sum-exp) and capture the target logit; then the weighted sum. */
int unok_row_lse_update(int dtype, int R, int Vc, const void* z, int64_t ldz, int c0,
                        const int64_t* tgt, float* run_max, float* run_sum, float* zt,
                        int first, void* stream);
int unok_ce_finish(int R, const float* run_max, const float* run_sum, const float* zt,
                   const float* w, const float* inv_n, float* lse, float* loss, void* stream);
int unok_ce_grad_chunk(int out_dtype, int R, int Vc, const float* z, int64_t ldz, int c0,
                       const float* lse, const int64_t* tgt, const float* w, const float* gscale,
                       const float* inv_n, void* dz, int64_t lddz, void* stream);
/* Cross-entropy over the LM head with the logit statistics formed in the GEMM's epilogue (the
 * loss of training/trainer.py:267-283 on the logits of training/losses.py:21-35). Z = H W^T with
 * H [R, K] bf16 (the CE rows' hidden states) and W [V, K] bf16 (LM-head rows vocab0 ..
 * vocab0 + V - 1); K a multiple of 64. Z is produced tile by tile inside the 256x256 MFMA GEMM; it
 * is written only when the caller asks for it.
 * unok_lmhead_ce_stats: pmax[r * ldp + b] / psum[r * ldp + b] = max / sum exp(z - max) over the
 *   columns [128 b, 128 b + 128) of row r (ldp >= ceil(V / 128)); zt[r] = Z[r, tgt[r] - vocab0]
 *   when the target lies in this product's columns; with z non-null also Z itself in fp32
 *   (z[r * ldz + v], ldz >= V and a multiple of 4, rows 16-byte aligned), for a backward that forms
 *   dz from the stored logits with unok_ce_grad_chunk instead of recomputing them.
 * unok_ce_parts_reduce: merges a row's blocks into run_max / run_sum (then unok_ce_finish).
 * unok_lmhead_ce_grad: dz[r, v] = bf16(w[r] * g * inv_n * (exp(Z[r, v] - lse[r]) - [vocab0 + v ==
 *   tgt[r]])) for one vocabulary chunk (g, inv_n device scalars), the operand of the data-gradient
 *   GEMM dH += dz W[chunk]. */
int unok_lmhead_ce_stats(int R, int V, int K, const void* H, int64_t ldh, const void* W, int64_t ldw,
                         const int64_t* tgt, int vocab0, float* pmax, float* psum, int64_t ldp,
                         float* zt, float* z, int64_t ldz, void* stream);
int unok_ce_parts_reduce(int R, int nparts, const float* pmax, const float* psum, int64_t ldp,
                         float* run_max, float* run_sum, void* stream);
int unok_lmhead_ce_grad(int R, int V, int K, const void* H, int64_t ldh, const void* W, int64_t ldw,
                        const int64_t* tgt, int vocab0, const float* lse, const float* w,
                        const float* g, const float* inv_n, void* dz, int64_t lddz, void* stream);
/* First-index argmax over vocab chunks: the "clean_argmax" CE target (training/losses.py:38-56). */
int unok_row_argmax_update(int dtype, int R, int Vc, const void* z, int64_t ldz, int c0,
                           float* best_val, int64_t* best_idx, int first, void* stream);
/* Total variation / reverse KL over full-vocabulary logits (training/losses.py:59-183). */
int unok_softmax_stats(int dtype, int R, int V, const void* z, int64_t ldz, float* mx, float* se,
                       void* stream);
int unok_tv_fwd(int dtype, int R, int V, const void* zs, int64_t lds, const void* zt, int64_t ldt,
                const float* ms, const float* ss, const float* mt, const float* st,
                float* row_l1, float* row_S, void* stream);
int unok_tv_bwd(int dtype, int R, int V, const void* zs, int64_t lds, const void* zt, int64_t ldt,
                const float* ms, const float* ss, const float* mt, const float* st,
                const float* row_S, const float* gscale, const float* inv_n, void* grad,
                int64_t ldg, void* stream);
int unok_kl_fwd(int dtype, int R, int V, const void* zs, int64_t lds, const void* zt, int64_t ldt,
                const float* ms, const float* ss, const float* mt, const float* st,
                float* row_kl, void* stream);
int unok_kl_bwd(int dtype, int R, int V, const void* zs, int64_t lds, const void* zt, int64_t ldt,
                const float* ms, const float* ss, const float* mt, const float* st,
                const float* row_kl, const float* gscale, const float* inv_n, void* grad,
                int64_t ldg, void* stream);
int unok_sum_scaled(int64_t n, const float* x, const float* inv_n, float* out, void* stream);

/* ---- Optimizer ------------------------------------------------------------------------------- */

/* Global L2 norm of the flat LoRA gradient and clip coefficient min(1, max/(norm+1e-6))
 * (torch.nn.utils.clip_grad_norm_ with max_grad_norm=1.0, training/train.py:287). */
int unok_grad_clip_coef(int64_t n, const float* g, float* partials, int nparts, float max_norm,
                        float* clip_out, void* stream);
/* torch.optim.AdamW step over the flat LoRA state (training/train.py:282-288), refreshing the
 * compute copy (B range scaled by alpha/r). */
int unok_adamw_step(int64_t n, float* p, float* g, float* m, float* v, const float* clip,
                    float lr, float beta1, float beta2, float eps, float weight_decay, int step,
                    int copy_dtype, void* copy, int64_t n_unscaled, float copy_scale,
                    void* stream);
int unok_cast_copy(int copy_dtype, int64_t n, int64_t n_unscaled, float scale, const float* p,
                   void* copy, void* stream);
int unok_transpose_jobs(int dtype, const int64_t* jobs, int njobs, int64_t total_tiles,
                        const void* src, void* dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* UNOK_H */
