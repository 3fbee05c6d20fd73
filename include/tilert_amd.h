/*
 * tilert_amd -- C ABI of the MI355X (gfx950) FP8 decode hot path.
 *
 * A plain C interface: device pointers, sizes and a hipStream_t passed as void*.
 * No torch types.  Every function is destination-passing (the caller owns every
 * output and workspace; the library never allocates) and returns an int status:
 *   0 = ok, 1 = bad argument, 2 = HIP launch error, 3 = unsupported shape/option;
 * on failure tl_last_error() returns a thread-local message.  Kernels are enqueued on
 * the given stream and never synchronise it.
 *
 * Conventions: fp8 = OCP float8_e4m3fn bytes; bf16 = uint16 bit patterns; block size
 * 128; activation scales fp32 [rows, K/128]; weight scales fp32 [ceil(N/128), K/128],
 * row-major weights [N, K].
 *
 * Reference interfaces replaced (paths relative to the tile-ai/TileRT tree):
 *   tl_act_quant        act_quant            tilert/models/deepseek_v3_2/refs/kernel.py:252-279
 *                       (fused form: rmsnorm_quant_op  .../ops/rmsnorm_quant.py:25-35)
 *   tl_weight_dequant   weight_dequant       .../refs/kernel.py:97-129
 *   tl_fp8_gemm         fp8_gemm             .../refs/kernel.py:282-306; the FP8 GEMVs behind
 *                       projx_wqkva_op (.../ops/projx_wqkva.py:22-48), rmsnorm_proj_qb_op,
 *                       unproj_o_allreduce_op, rmsnorm_up_gate_silu_op, down_allreduce_op
 *   tl_fp8_pack_weight  the per-op weight converters (load-time layout change)
 *   tl_projx_wqkva      projx_wqkva_op       .../ops/projx_wqkva.py:22-48 (golden :268-294)
 *   tl_rmsnorm_projq_wqb  rmsnorm_proj_qb_op  .../ops/rmsnorm_projq_wqb.py:20-44 (golden :496-512)
 *   tl_moe_gate_up_swiglu  expert_select_up_gate_silu_op  .../ops/expert_sel_up_gate_silu.py:23-48
 *   tl_moe_down_combine    expert_down_allreduce_op       .../ops/expert_down_allreduce.py:23-63
 *                          (these two: config 2's expert-parallel shard, routing as input)
 *   tl_moe_route           routing of expert_select_up_gate_silu_op (golden _ref_expert_select_ds,
 *                          glm_5/_dsa_v32/ops/expert_sel_up_gate_silu.py:714-737)
 *   tl_expert_select_up_gate_silu  expert_select_up_gate_silu_op  .../ops/expert_sel_up_gate_silu.py:23-48
 *   tl_expert_down_allreduce       expert_down_allreduce_op       .../ops/expert_down_allreduce.py:23-63
 *                          (these two: the reference's own tensor-parallel layout, shared expert)
 *   tl_head_gemm_bf16        projq_wqb_op / projo_wkvb_op / unproj_o_allreduce_op
 *                            .../ops/projq_wqb.py:24-54, projo_wkvb.py:24-54, unproj_o_allreduce.py:23-58
 *   tl_projx_wqaki           projx_wqaki_op           .../ops/projx_wqaki.py:11-44
 *   tl_bf16_gemv             proj_w_op (projx_wis)    .../ops/projx_wis.py:18-37
 *   tl_rmsnorm_projq_wqb with rope_dim = 0: rmsnorm_proj_qi_op  .../ops/rmsnorm_projq_wqi.py:17-37
 *   tl_rmsnorm_up_gate_silu  rmsnorm_up_gate_silu_op  .../ops/rmsnorm_up_gate_silu.py:26-44
 *   tl_down_allreduce        down_allreduce_op        .../ops/down_allreduce.py:24-59
 *   tl_rmsnorm_quant       rmsnorm_quant_op / rmsnorm_op  .../ops/rmsnorm_quant.py:19-63
 *   tl_indexer_fp8_scores  sparse_index_op                .../ops/sparse_index.py:11-69
 *   tl_indexer_fp8_scores_paged  the same over KI pages    pd_vllm/profiles/mla_nsa.py:211-228
 *   tl_ki_cache_write      writer of the KI page format    pd_vllm/profiles/mla_nsa.py:17-41
 *   tl_layernorm_rope_rotate     layernorm_rope_rotate_op  .../ops/layernorm_rope_rotate.py:23-82
 *                                (golden :206-220)
 *   tl_layernorm_rope_rotate_ki  the same, its keys quantised into KI pages (the producer of
 *                                the format tl_indexer_fp8_scores_paged reads)
 *   tl_flash_sparse_mla    flash_sparse_mla_op            .../ops/flash_sparse_mla.py:18-93
 *                          (golden FlashSparseMLACombine.golden_forward :152-196)
 *   tl_topk_rows           topk_accurate_op               .../ops/topk.py:62-109
 *   tl_indexer_fp8_topk    sparse_index_topk_dsv32_op (fp8 cache)  .../ops/sparse_index.py:72-128
 *   tl_indexer_bf16_scores sparse_index_op (bf16, the reference's own)  .../ops/sparse_index.py:11-69
 *   tl_indexer_bf16_topk   sparse_index_topk_dsv32_op  .../ops/sparse_index.py:72-128 and
 *                          sparse_index_topk_glm5_v3_op  glm_5/ops/sparse_index_v3.py:10-51
 */
#ifndef TILERT_AMD_H_
#define TILERT_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scale_mode values for tl_act_quant */
#define TL_SCALE_REFERENCE 0 /* s = max(amax,1e-4) * fp32(1/448)   refs/kernel.py:191 */
#define TL_SCALE_UE8M0 1     /* s = 2^ceil(log2(max(amax,1e-4)/448)) refs/kernel.py:140-151 */
#define TL_SCALE_DIV 2       /* s = max(amax,1e-4) / 448 (IEEE division) */

const char* tl_last_error(void);
const char* tl_version(void);

/* Per-(row, 128-column group) quantisation of bf16 x [rows, K] to e4m3fn y [rows, K] with
 * fp32 scales s [rows, K/128]: y = e4m3(clamp(x / s, -448, 448)), RNE, IEEE division.
 * group must be 128.  Replaces act_quant (refs/kernel.py:252-279). */
int tl_act_quant(const void* x_bf16, void* y_fp8, float* s, int64_t rows, int64_t K,
                 int64_t group, int scale_mode, void* stream);

/* 128x128 block quantisation of a weight w [N, K] (fp32, or bf16 when w_is_bf16):
 * s = block_amax / 448 (1 for an all-zero block), q = e4m3(clamp(w / s)).  Weight
 * preparation (the per-op converters' job in the reference, e.g. convert_to_mma in
 * expert_sel_up_gate_silu.py); not on the per-token path. */
int tl_weight_quant(const void* w, int w_is_bf16, void* q_fp8, float* s, int64_t N, int64_t K,
                    void* stream);

/* out[n,k] = fp32(q[n,k]) * s[n/128, k/128], written as fp32 or bf16 (out_bf16 = 1).
 * Replaces weight_dequant / _weight_dequant_torch (refs/kernel.py:82-129). */
int tl_weight_dequant(const void* q_fp8, const float* s, void* out, int out_bf16, int64_t N,
                      int64_t K, void* stream);

/* c[M,N] bf16 = (a . b^T) with per-128-K-block scaling, fp32 accumulation.
 * a fp8 [M,K], a_s fp32 [M,K/128], b fp8 [N,K], b_s fp32 [ceil(N/128),K/128].
 * Requires K % 128 == 0, N % 16 == 0, 1 <= M <= 256, 16-byte aligned a and b.
 * From M = 16 on (a rearranged copy of the activations, or the packed MFMA GEMM's split-K
 * partials from M = 17 or 33) and for narrow layers at M > 16 (split-K partials) the call needs
 * a workspace of tl_fp8_gemm_workspace_bytes(M,N,K)
 * bytes (0 = none), ZERO-FILLED before its first use; the kernels leave it ready for the
 * next call.  Calls that share a workspace must be ordered
 * (same stream).  Replaces fp8_gemm (refs/kernel.py:282-306). */
size_t tl_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);
int tl_fp8_gemm(const void* a, const float* a_s, const void* b, const float* b_s, void* c_bf16,
                int64_t M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                void* stream);

/* Repack a canonical fp8 weight [N, K] (N % 16 == 0, K % 512 == 0) into MFMA operand
 * fragments for tl_fp8_gemm_packed.  Fragment (t, kb) -- rows 16t..16t+15, columns
 * 128kb..128kb+127 -- is 2048 contiguous bytes at fragment index
 * ((kb / 4) * (N/16) + t) * 4 + kb % 4 ("K-group-major": a workgroup's 4 K blocks per step
 * are 8 KB of consecutive memory and neighbouring row tiles are neighbours); within it,
 * byte p*1024 + l*16 + i (piece p in {0,1}, lane l in [0,64), i in [0,16)) is
 * W[16 t + (l % 16)][128 kb + 64 p + 16 (l / 16) + i].  packed must hold N*K bytes and not
 * alias b.  Counterpart of the reference's per-op weight converters (e.g.
 * RMSNormProjQKVAFP8MMAWeightsConverter, rmsnorm_projx_wqkva.py:18-119): a one-time,
 * load-time layout change. */
int tl_fp8_pack_weight(const void* b, void* packed, int64_t N, int64_t K, void* stream);

/* tl_fp8_gemm with b in the fragment-packed layout of tl_fp8_pack_weight (same scales,
 * same workspace rule).  Results equal tl_fp8_gemm's bit for bit where both run the GEMV
 * (M <= 16, or N % 128 != 0); from M = 17 or 33 with N % 128 == 0 the packed layout runs an MFMA
 * GEMM that sums the K blocks in another order (same tolerance against the reference).
 * The FP8 GEMV / GEMM behind the reference's packed-weight projection ops (projx_wqkva_op,
 * rmsnorm_up_gate_silu_op, ...). */
int tl_fp8_gemm_packed(const void* a, const float* a_s, const void* b_packed, const float* b_s,
                       void* c_bf16, int64_t M, int64_t N, int64_t K, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Allocation-free variant of tl_fp8_gemm_packed -- NO COUNTERPART IN THE REFERENCE.  For
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the same kernels and results (bit for bit), with
 * their scratch (split-K counters and partials, the activation image) in a static device
 * array of TL_FP8_GEMM_STATIC_SCRATCH_BYTES that each GPU holds until the process ends,
 * instead of a workspace argument.  The call allocates nothing; shapes whose scratch would
 * exceed the maximum fail with status 3 (every dense MLP shape of 7168 <-> 18432 up to
 * M = 256 fits).  Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, or different threads without ordering) race; calls on one stream are
 * safe.  The array is zero when the library's code object loads and every call leaves its
 * counters zero again, so no call clears it (a first call may be made under graph
 * capture).  The 40 MiB are reserved on every GPU where the library's code object is
 * loaded, whether or not this entry point is called. */
#define TL_FP8_GEMM_STATIC_SCRATCH_BYTES (40u << 20)
int tl_fp8_gemm_packed_static(const void* a, const float* a_s, const void* b_packed, const float* b_s,
                              void* c_bf16, int64_t M, int64_t N, int64_t K, void* stream);

/* The fused attention down-projection of one decode step: x_q . [wq_a; wkv_a]^T in one
 * launch, its columns routed to three outputs.  x_q fp8 [batch*seq, dim] + x_s fp32
 * [batch*seq, dim/128]; w_packed = tl_fp8_pack_weight of the row-stacked weight
 * [q_rank + kv_rank + rope_dim, dim] (wq_a, then wkv_a = kv_a_proj_with_mqa: kv_rank latent
 * rows, then rope_dim rope rows), w_s its fp32 block scales [ceil(N/128), dim/128] (wq_a's
 * scale rows, then wkv_a's: q_rank % 128 == 0 makes the stack an ordinary block-scaled
 * weight).  Outputs bf16: q_out [batch*seq, q_rank], kv_out [batch*seq, kv_rank], and the
 * rope part written into pe_cache [batch, cache_rows, rope_dim] at row *cur_pos + s for
 * token (b, s) (cur_pos: device int32, read by the kernel; rows outside [0, cache_rows)
 * are not written).  Needs batch*seq <= 64, dim % 512 == 0, kv_rank and rope_dim multiples
 * of 16, and the workspace of tl_fp8_gemm_workspace_bytes(batch*seq, N, dim).  Replaces
 * projx_wqkva_op (tilert/models/deepseek_v3_2/ops/projx_wqkva.py:22-48; golden :268-294). */
int tl_projx_wqkva(const void* x_q, const float* x_s, const void* w_packed, const float* w_s,
                   const int32_t* cur_pos, void* q_out, void* kv_out, void* pe_cache,
                   int64_t batch, int64_t seq, int64_t cache_rows, int64_t dim, int64_t q_rank,
                   int64_t kv_rank, int64_t rope_dim, void* workspace, size_t workspace_bytes,
                   void* stream);

/* Tile-major fragment packing for the MoE kernels: the stacked per-expert weights
 * [rows, K] (rows % 16 == 0, K % 128 == 0) become fragments (t, kb) at (t*K/128 + kb)*2048
 * with the in-fragment order of tl_fp8_pack_weight.  Load-time layout change (the role of
 * ExpertSelectUpGateSiLUWeightsConverter / the down converters in the reference). */
int tl_moe_pack_weight(const void* b, void* packed, int64_t rows, int64_t K, void* stream);

/* MoE gate/up + SwiGLU at one expert-parallel shard (bf16 activations x fp8 weights,
 * the reference MoE's BF16MMA numerics).
 * x bf16 [M, D]; w13_packed = tl_moe_pack_weight of the stacked per-expert gate/up
 * weights [n_local * 2I, D] (expert e: rows e*2I .. e*2I+I-1 gate, then I rows up);
 * s13 fp32 [n_local, 2I/128, D/128].  topk_idx int32 [M, topk] holds global expert ids;
 * the shard owns ids [expert_begin, expert_begin + n_local).  Every local expert hit by
 * at least one token gets a slot (ascending expert order); h bf16 [n_local, M, I]
 * receives, for slot s < n_hit and EVERY token t,
 *   h[s,t,:] = bf16(silu(x_t . G^T) * (x_t . U^T))  (fp32 products and SwiGLU),
 * where G, U are the block-dequantised weights; rows of unrouted tokens are computed but
 * ignored by tl_moe_down_combine; slots >= n_hit are not written.
 * 1 <= M <= 16, n_local <= 64, D and I multiples of 128.
 * Replaces the grouped GEMM of expert_select_up_gate_silu_op
 * (deepseek_v3_2/ops/expert_sel_up_gate_silu.py:23-48, golden :670-692); routing is an
 * input. */
int tl_moe_gate_up_swiglu(const void* x_bf16, const void* w13_packed, const float* s13,
                          const int32_t* topk_idx, int64_t M, int64_t topk, int64_t expert_begin,
                          int64_t n_local, int64_t D, int64_t I, void* h_bf16, void* stream);

/* MoE down projection + routing-weighted combine at one shard.
 * h bf16 [n_local, M, I] from tl_moe_gate_up_swiglu (same topk_idx); w2_packed =
 * tl_moe_pack_weight of the stacked down weights [n_local * D, I]; s2 fp32
 * [n_local, D/128, I/128]; topk_w fp32 [M, topk].
 *   y[t] = bf16( sum over the token's local experts e, ascending, of
 *                bf16(w[t,e] * (h[t,e] . D_e^T)) )   (fp32 sum)
 * y bf16 [M, D]; 0 for tokens with no local expert (the shard's partial of the
 * allreduce).  Replaces expert_down_allreduce_op
 * (deepseek_v3_2/ops/expert_down_allreduce.py:23-63, golden :455-468) without the
 * cross-GPU allreduce. */
int tl_moe_down_combine(const void* h_bf16, const void* w2_packed, const float* s2,
                        const int32_t* topk_idx, const float* topk_w, int64_t M, int64_t topk,
                        int64_t expert_begin, int64_t n_local, int64_t D, int64_t I,
                        void* y_bf16, void* stream);

/* ---- The reference's MoE and dense-MLP operators in their own layout: one device's share of
 * the tensor-parallel split of every expert's intermediate dim (I rows per expert).  Local
 * expert 0 is the shared expert, 1 + j routed expert j.  Weights: tl_moe_pack_weight of the
 * stacked [n_local * 2I, D] gate/up (per expert I gate rows, then I up rows) and
 * [n_local * D, I] down matrices; fp32 block scales [n_local, 2I/128, D/128] and
 * [n_local, D/128, I/128].  bf16 activations times bf16(fp32(q) * scale) weights, fp32
 * accumulation (the goldens' bf16 reference weights).  1 <= M <= 16 tokens (one 16-row MFMA
 * tile), at most 64 (token, position) pairs, x [M, D] within 64 KB (M <= 4 at D = 7168).
 * With a bias and n_groups > 1 every group holds >= 2 experts. */

/* Routing of expert_select_up_gate_silu_op (golden _ref_expert_select_ds,
 * glm_5/_dsa_v32/ops/expert_sel_up_gate_silu.py:714-737; n_groups = 1 is
 * _ref_expert_select_glm5, deepseek_v3_2/ops/expert_sel_up_gate_silu.py:641-652):
 * scores fp32 [M, n_routed] router logits, bias fp32 [n_routed] (nullable): s = sigmoid,
 * choice on s + bias, limited to the topk_groups best of n_groups groups (score: the sum of
 * a group's two largest biased scores; its largest without bias), top-k in descending
 * order (lowest id first on ties); probs_out [M, topk] = the chosen s / their sum *
 * route_scale, idx_out int32 [M, topk].  n_routed <= 256. */
int tl_moe_route(const float* scores, const float* bias, int64_t M, int64_t n_routed, int64_t topk,
                 int64_t n_groups, int64_t topk_groups, float route_scale, float* probs_out,
                 int32_t* idx_out, void* stream);

/* expert_select_up_gate_silu_op (deepseek_v3_2/ops/expert_sel_up_gate_silu.py:23-48; golden
 * :654-692): tl_moe_route, then for every token t and position p (0 = shared expert,
 * 1 + j = its j-th selected expert) h[t, p, :] = bf16(silu(x_t . G^T) * (x_t . U^T)).
 * x bf16 [M, D]; h bf16 [M, 1 + topk, I]; probs_out / idx_out as tl_moe_route.  One
 * launch (every gate/up workgroup routes the M tokens itself; workgroup 0 writes probs_out
 * and idx_out); only the hit experts' weights are read. */
int tl_expert_select_up_gate_silu(const void* x_bf16, const float* scores, const float* bias,
                                  const void* w13_packed, const float* s13, int64_t M, int64_t n_routed,
                                  int64_t topk, int64_t n_groups, int64_t topk_groups, float route_scale,
                                  int64_t D, int64_t I, void* h_bf16, float* probs_out, int32_t* idx_out,
                                  void* stream);

/* expert_down_allreduce_op (deepseek_v3_2/ops/expert_down_allreduce.py:23-63; golden
 * :445-468) at one device: h bf16 [M, 1 + topk, I] (tl_expert_select_up_gate_silu's), idx
 * int32 / probs fp32 [M, topk] (distinct ids per token; ids outside [0, n_routed) are
 * skipped): y[t] = bf16( sum_p bf16(w[t,p] * (h[t,p] . D_{e(t,p)}^T)) ), w = 1 for the
 * shared position, fp32 sum; when x_in bf16 [M, D] is given, y = bf16(y + x_in) (the
 * allreduce epilogue's residual; across devices the partials would be summed first).
 * y bf16 [M, D]. */
int tl_expert_down_allreduce(const void* h_bf16, const void* w2_packed, const float* s2, const int32_t* idx,
                             const float* probs, const void* x_in_bf16, int64_t M, int64_t n_routed,
                             int64_t topk, int64_t D, int64_t I, void* y_bf16, void* stream);

/* rmsnorm_up_gate_silu_op (deepseek_v3_2/ops/rmsnorm_up_gate_silu.py:26-44; golden
 * :318-347): the dense MLP's device share as n_chunks chunks of I rows (chunk i = the
 * reference's pseudo-expert i).  xn = bf16(x * 1/sqrt(mean(x^2) + eps) * gamma) in fp32,
 * then h[t, i, :] = bf16(silu(xn_t . G_i^T) * (xn_t . U_i^T)).  x bf16 [M, D], gamma fp32
 * [D] (16-byte aligned), h bf16 [M, n_chunks, I].  One launch. */
int tl_rmsnorm_up_gate_silu(const void* x_bf16, const float* gamma, float eps, const void* w13_packed,
                            const float* s13, int64_t M, int64_t n_chunks, int64_t D, int64_t I, void* h_bf16,
                            void* stream);

/* down_allreduce_op (deepseek_v3_2/ops/down_allreduce.py:24-59; golden :293-320):
 * y[t] = bf16( sum_i bf16(h[t,i] . D_i^T) ) (+ x_in as tl_expert_down_allreduce).
 * h bf16 [M, n_chunks, I], y bf16 [M, D]. */
int tl_down_allreduce(const void* h_bf16, const void* w2_packed, const float* s2, const void* x_in_bf16,
                      int64_t M, int64_t n_chunks, int64_t D, int64_t I, void* y_bf16, void* stream);

/* Per-head bf16 x fp8 GEMV: y[t, h, :] = bf16(x[t, h, :] . W_h^T) for H weights W_h [N, K]
 * (bf16 activations times bf16(fp32(q) * block scale) weights, fp32 accumulation), and
 * y = bf16(y + x_in) when x_in bf16 [M, H, N] is given.  x bf16 [M, H, K] (M*H*K*2 <= 64 KB),
 * w_packed = tl_moe_pack_weight of the stacked [H * N, K] weights, w_s fp32
 * [H, ceil(N/128), K/128], y bf16 [M, H, N]; N % 16 == 0, K % 128 == 0, M <= 16.  The absorbed
 * MLA projections at one device's share: projq_wqb_op (.../ops/projq_wqb.py:24-54, golden
 * :448-450; each head's [128, kv_lora] nope block of wkv_b stored transposed), projo_wkvb_op
 * (.../ops/projo_wkvb.py:24-54, golden :465-467) and, with H = 1 and the residual,
 * unproj_o_allreduce_op (.../ops/unproj_o_allreduce.py:23-58, golden :480-498; the single-GPU
 * form of its allreduce epilogue). */
int tl_head_gemm_bf16(const void* x_bf16, const void* w_packed, const float* w_s, const void* x_in_bf16,
                      int64_t M, int64_t H, int64_t N, int64_t K, void* y_bf16, void* stream);

/* The indexer's fused query/key down-projection, projx_wqaki_op
 * (deepseek_v3_2/ops/projx_wqaki.py:11-44): x_q . [wq_a; wk]^T in one FP8 GEMV launch, columns
 * [0, q_rank) -> q_out bf16 [M, q_rank], the rest -> ki_out bf16 [M, ki_dim].  w_packed =
 * tl_fp8_pack_weight of the row-stacked [q_rank + ki_dim, dim] weight, w_s its fp32 block
 * scales (wq_a's rows, then wk's; q_rank % 128 == 0).  M <= 64, dim % 512 == 0; workspace
 * as tl_fp8_gemm_workspace_bytes(M, q_rank + ki_dim, dim). */
int tl_projx_wqaki(const void* x_q, const float* x_s, const void* w_packed, const float* w_s, void* q_out,
                   void* ki_out, int64_t M, int64_t dim, int64_t q_rank, int64_t ki_dim, void* workspace,
                   size_t workspace_bytes, void* stream);

/* y bf16 [M, N] = bf16(x . w^T) with bf16 x [M, K] and bf16 weights w [N, K] (row-major),
 * fp32 accumulation: proj_w_op, the indexer head-weight projection of projx_wis
 * (deepseek_v3_2/ops/projx_wis.py:18-37; golden RMSNormProjxWqakis :289-299).  M <= 16,
 * N % 16 == 0 (N <= 262144), K % 128 == 0 (K <= 65536).  K is split over workgroups: the
 * workspace (tl_bf16_gemv_workspace_bytes; 0 bytes when K <= 512) is the zero-initialised
 * split-K workspace of tl_fp8_gemm -- its counter region is left zero by every call, so
 * one buffer per stream serves both. */
size_t tl_bf16_gemv_workspace_bytes(int64_t M, int64_t N, int64_t K);
int tl_bf16_gemv(const void* x_bf16, const void* w_bf16, int64_t M, int64_t N, int64_t K, void* y_bf16,
                 void* workspace, size_t workspace_bytes, void* stream);

/* RMSNorm with optional activation quantisation (rmsnorm_quant_op / rmsnorm_op,
 * ops/rmsnorm_quant.py:19-63; norm of tilert/models/common.py:92-133 without residual).
 * x bf16 [rows, dim], gamma fp32 [dim]: y_bf16 = bf16(gamma * x * 1/sqrt(mean(x^2) + eps))
 * (fp32 math); when y_fp8 / y_scale are non-null, they receive act_quant of y_bf16 per
 * 1x128 group (fp8 e4m3fn [rows, dim], fp32 [rows, dim/128], scale_mode as
 * tl_act_quant) -- bit-identical to tl_act_quant applied to y_bf16.  dim % 128 == 0,
 * dim <= 16384; pointers 16-byte aligned. */
int tl_rmsnorm_quant(const void* x_bf16, const float* gamma, float eps, int64_t rows, int64_t dim,
                     void* y_bf16, void* y_fp8, float* y_scale, int scale_mode, void* stream);

/* DSA lightning-indexer scores over an fp8 key cache.
 * q fp8 [M, H, 128]; q_s fp32 per token [M] (q_s_per_head = 0) or per (token, head)
 * [M, H] (q_s_per_head = 1); k fp8 [L, 128]; k_s fp32 [L]; w bf16 [M, H].
 * logits fp32 [M, ld] (ld >= L): logits[t,l] = sum_h w[t,h]*ReLU(qd[t,h].kd[l]) for
 * l <= cur_pos + t, -inf for cur_pos + t < l < L.  H in {32, 64}, M*H <= 256.
 * Replaces sparse_index_op (ops/sparse_index.py:11-69) for an fp8 cache. */
int tl_indexer_fp8_scores(const void* q_fp8, const float* q_s, int q_s_per_head,
                          const void* k_fp8, const float* k_s, const void* w_bf16,
                          float* logits, int64_t M, int64_t H, int64_t L, int64_t ld,
                          int64_t cur_pos, void* stream);

/* Paged variant: the key cache in pd_vllm's KI page layout
 * (pd_vllm/profiles/mla_nsa.py:17-41,211-228): ki_pages u8 [n_pages, 8448], page p =
 * 64 keys x 128 fp8 (8192 B) followed by their 64 fp32 scales (256 B); key l lives in
 * page l / 64, row l % 64.  L <= 64 * n_pages; pages 16-byte aligned.  Bit-identical to
 * tl_indexer_fp8_scores on the equivalent flat cache.  Replaces sparse_index_op's cache
 * read (ops/sparse_index.py:11-69) for the cache format MlaNsaProfile._dequant_ki reads. */
int tl_indexer_fp8_scores_paged(const void* q_fp8, const float* q_s, int q_s_per_head,
                                const void* ki_pages, int64_t n_pages, const void* w_bf16,
                                float* logits, int64_t M, int64_t H, int64_t L, int64_t ld,
                                int64_t cur_pos, void* stream);

/* sparse_index_topk as one call (sparse_index_topk_dsv32_op, ops/sparse_index.py:72-128; the
 * selection is topk_accurate's, ops/topk.py:62-109): the scores of tl_indexer_fp8_scores into
 * logits, then on the same stream indices int32 [M, topk] = the exact top-topk key positions
 * of each token's visible keys 0 .. cur_pos + t, ascending, ties at the threshold to the
 * lowest positions, -1 past the visible count (tl_topk_rows with valid_base = cur_pos).
 * topk <= 8192, ld % 4 == 0, ld <= 262144, logits 16-byte aligned.  workspace: at least
 * tl_indexer_topk_workspace_bytes(M, ld, topk) bytes (= tl_topk_workspace_bytes), zero-filled
 * once before its first use; every call leaves it reusable, so calls of any shapes in stream
 * order may share one (calls that overlap on one workspace race). */
size_t tl_indexer_topk_workspace_bytes(int64_t M, int64_t ld, int64_t topk);
int tl_indexer_fp8_topk(const void* q_fp8, const float* q_s, int q_s_per_head, const void* k_fp8,
                        const float* k_s, const void* w_bf16, float* logits, int64_t M, int64_t H,
                        int64_t L, int64_t ld, int64_t cur_pos, int64_t topk, int32_t* indices,
                        void* workspace, size_t workspace_bytes, void* stream);

/* The reference's bf16 indexer (sparse_index_op, ops/sparse_index.py:11-69): q bf16
 * [M, H, 128], k bf16 [L, 128] (the index-key cache), w bf16 [M, H]; logits[t, l] =
 * score_scale * sum_h w[t,h] * ReLU(q[t,h] . k[l]) in fp32 (bf16 MFMA) for l <= cur_pos + t,
 * -inf for cur_pos + t < l < L.  H in {32, 64}, M*H <= 256; q, k 16-byte aligned. */
int tl_indexer_bf16_scores(const void* q_bf16, const void* k_bf16, const void* w_bf16, float score_scale,
                           float* logits, int64_t M, int64_t H, int64_t L, int64_t ld, int64_t cur_pos,
                           void* stream);

/* tl_indexer_bf16_scores and the top-k of tl_indexer_fp8_topk as one call:
 * sparse_index_topk_dsv32_op (H = 64, ops/sparse_index.py:72-128) and
 * sparse_index_topk_glm5_v3_op (H = 32, glm_5/ops/sparse_index_v3.py:10-51). */
int tl_indexer_bf16_topk(const void* q_bf16, const void* k_bf16, const void* w_bf16, float score_scale,
                         float* logits, int64_t M, int64_t H, int64_t L, int64_t ld, int64_t cur_pos,
                         int64_t topk, int32_t* indices, void* workspace, size_t workspace_bytes,
                         void* stream);

/* Write `rows` keys (bf16 [rows, 128]) into KI pages at positions pos .. pos+rows-1:
 * per key s = the act_quant group scale of its amax (scale_mode as tl_act_quant), fp8 =
 * e4m3fn(clamp(k / s, +-448)), stored at page (pos+i) / 64, row (pos+i) % 64, its scale
 * after the page's fp8 block.  The producer side of the format MlaNsaProfile._dequant_ki
 * reads (mla_nsa.py:211-228); the key rotation of layernorm_rope_rotate
 * (ops/layernorm_rope_rotate.py:206-220) happens upstream.  pos + rows <= 64 * n_pages. */
int tl_ki_cache_write(const void* k_bf16, int64_t rows, void* ki_pages, int64_t n_pages, int64_t pos,
                      int scale_mode, void* stream);

/* RMSNorm of the q latent + wq_b, RmsnormProjqWqb (ops/rmsnorm_projq_wqb.py:20-44, golden
 * :496-512, BF16MMA): qr = bf16(q * rsqrt(mean(q^2) + eps) * q_norm_weight) in fp32 for the M
 * rows of q bf16 [M, q_rank]; out = qr . W^T with W = bf16(fp32(wq_b) * block scale) (the
 * golden's bf16 dequantised weight), fp32 accumulation, bf16 result, written per head as
 * q_nope [M, heads, nope_dim] and q_pe [M, heads, rope_dim] (feature h * (nope + rope) + d
 * of the weight is head h, dim d).  wq_b_packed: the [heads * (nope + rope), q_rank] e4m3fn
 * weight in tl_fp8_pack_weight's layout; wq_b_s its fp32 [N/128, q_rank/128] scales.
 * 1 <= M <= 16, q_rank % 512 == 0 and <= 2048, nope/rope multiples of 16.  rope_dim = 0 sends
 * every feature to q_nope (q_pe may be null): rmsnorm_proj_qi_op, the indexer's query
 * projection (ops/rmsnorm_projq_wqi.py:17-37, golden :301-314), heads = 64, nope = 128. */
int tl_rmsnorm_projq_wqb(const void* q_bf16, const float* q_norm_weight, float eps, const void* wq_b_packed,
                         const float* wq_b_s, void* q_nope_bf16, void* q_pe_bf16, int64_t M, int64_t heads,
                         int64_t q_rank, int64_t nope_dim, int64_t rope_dim, void* stream);

/* Indexer key producer, LayerNormRoPERotate (ops/layernorm_rope_rotate.py:23-82, golden
 * :206-220): for each of `seq` bf16 keys x [seq, 128], k = bf16(LayerNorm(x) * weight +
 * bias) with fp32 statistics and the given eps (the golden's 1e-6); dims 0..63 take the
 * non-interleaved RoPE (element i pairs with i + 32, times the complex freqs[t, i]; freqs is
 * fp32 [seq, 64] = (cos, sin) interleaved, the op's view_as_real of freqs_cis), rounded to
 * bf16; then the 128-point Hadamard transform scaled by 128^-1/2 (rotate_activation,
 * ops/rotate.py:17-21), rounded to bf16.  weight, bias fp32 [128].  Key t is written to row
 * *cur_pos + t (cur_pos: device int32) of k_cache_bf16 [cache_rows, 128]; rows outside the
 * cache are dropped.  Replaces layernorm_rope_rotate_op. */
int tl_layernorm_rope_rotate(const void* x_bf16, int64_t seq, const int32_t* cur_pos, void* k_cache_bf16,
                             int64_t cache_rows, const float* weight, const float* bias, const float* freqs,
                             float eps, void* stream);

/* The same keys quantised straight into KI pages (uint8 [n_pages, 8448]) at positions
 * *cur_pos + t, exactly as tl_ki_cache_write would store the bf16 result (scale_mode as
 * tl_act_quant): the producer of the page cache tl_indexer_fp8_scores_paged reads, with no
 * bf16 round trip through memory.  Positions outside the pages are dropped. */
int tl_layernorm_rope_rotate_ki(const void* x_bf16, int64_t seq, const int32_t* cur_pos, void* ki_pages,
                                int64_t n_pages, const float* weight, const float* bias, const float* freqs,
                                float eps, int scale_mode, void* stream);

/* Sparse MLA decode attention over the indexer's selection, flash_sparse_mla_op
 * (ops/flash_sparse_mla.py:18-93; golden :152-196).  q_nope bf16 [seqlen, heads, 512],
 * q_pe bf16 [seqlen, heads, 64], kv bf16 [kv_rows, 512], pe bf16 [kv_rows, 64], indices int32
 * [seqlen, topk] (distinct positions; entries outside [0, kv_rows) are ignored), cur_pos
 * device int32.  For token s and head h: softmax over the selected positions t of
 * (q_nope . kv[t] + q_pe . pe[t]) * softmax_scale (fp32; for seqlen > 1 positions after
 * *cur_pos + s are masked too), probabilities as bf16, times kv[t], fp32 accumulation ->
 * out bf16 [seqlen, heads, 512].  Split-K over ceil(topk / 64) <= 32 splits of 64 positions:
 * out_acc fp32 [seqlen, heads, 32, 512] receives each split's normalised output, lse_acc
 * fp32 [seqlen, heads, 32] its ln-sum-exp (-inf for a split with nothing visible), lse fp32
 * [seqlen, heads] the total (the reference op's output_acc / lse_acc / lse; a token with no
 * visible position gets zeros and -inf).  1 <= seqlen <= 16, 1 <= heads <= 32,
 * 1 <= topk <= 2048. */
int tl_flash_sparse_mla(const void* q_nope_bf16, const void* q_pe_bf16, const void* kv_bf16,
                        const void* pe_bf16, const int32_t* indices, const int32_t* cur_pos,
                        int64_t seqlen, int64_t heads, int64_t topk, int64_t kv_rows,
                        float softmax_scale, void* out_bf16, float* out_acc, float* lse,
                        float* lse_acc, void* stream);

/* Exact per-row top-k.  logits fp32 [rows, ld]; row i considers columns
 * [0, valid_base + 1 + i) (clamped to [0, ld]) -- topk_accurate's convention with
 * valid_base = seq_len - num_samples (ops/topk.py:77-80,101).  out int32 [rows, k]
 * receives the k selected column indices in ASCENDING INDEX order: every column whose
 * score is above the k-th largest, plus the lowest-index columns equal to it; when a
 * row has fewer than k valid columns, all of them, then -1.  The selected set is exactly
 * torch.topk's (ops/topk.py:128-143) up to the choice among exact ties, which is
 * lowest-index-first here.  1 <= k <= 8192.  workspace: tl_topk_workspace_bytes(rows,
 * ld, k) bytes, ZERO-FILLED before first use and left zeroed by every call (the state
 * that must be zero has fixed offsets, so calls of any shapes may share one workspace);
 * calls sharing it must be ordered.  Replaces topk_accurate_op (ops/topk.py:62-109). */
size_t tl_topk_workspace_bytes(int64_t rows, int64_t ld, int64_t k);
int tl_topk_rows(const float* logits, int64_t rows, int64_t ld, int64_t valid_base, int64_t k,
                 int32_t* out, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TILERT_AMD_H_ */
