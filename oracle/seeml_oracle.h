/*
 * seeml_oracle.h — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of SeeML's CPU executor kernel library
 * (runtime/executor/*.cc in the reference) and of its op-dispatch loop
 * (UpdateEngine::ExecuteRange, runtime/engine/update_engine.cc:306-509).
 * It is the checker the HIP backend is measured against: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * Nothing in the product path links or calls it.
 *
 * Each function names the reference file:line it restates. Expression order,
 * accumulator types (double partials) and ParallelFor chunk geometry follow
 * the reference exactly, so with -ffp-contract=off the results are
 * bit-identical to the reference kernels (pinned by tests against
 * oracle/_ref, the reference's own sources compiled in place).
 */
#ifndef SEEML_ORACLE_H_
#define SEEML_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ParallelChunkGrain / ParallelChunkCount (source/parallel/parallel_for.h:55-67). */
size_t orc_chunk_grain(size_t n, size_t grain);
size_t orc_chunk_count(size_t n, size_t grain);

/* GEMM family (runtime/executor/gemm.cc). act: 0 none, 1 relu, 2 gelu, 3 silu. */
void orc_gemm_nn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* bias, int act);
void orc_gemm_nt(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K);
void orc_gemm_tn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K);
void orc_gemm_acc_nn(const float* A, const float* B, float* C, size_t M,
                     size_t N, size_t K, float alpha);
void orc_gemm_nn_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale, int act);
void orc_gemm_nt_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale);

/* Elementwise / activation (elementwise.cc, activation.cc). */
void orc_add_ew(const float* x, const float* y, float* out, size_t n);
void orc_mul_ew(const float* x, const float* y, float* out, size_t n);
void orc_add_bias(const float* x, const float* b, float* out, size_t rows,
                  size_t cols);
void orc_scale(const float* x, float* out, float alpha, size_t n);
void orc_reduce_rows(const float* dy, float* db, size_t rows, size_t cols);
void orc_relu_fwd(const float* x, float* out, size_t n);
void orc_relu_bwd(const float* dy, const float* x, float* dx, size_t n);
void orc_gelu_fwd(const float* x, float* out, size_t n);
void orc_gelu_bwd(const float* dy, const float* x, float* dx, size_t n);
void orc_silu_fwd(const float* x, float* out, size_t n);
void orc_silu_bwd(const float* dy, const float* x, float* dx, size_t n);
void orc_embed_fwd(const int32_t* tokens, const float* table, float* out,
                   size_t rows, size_t dim);
void orc_fill(float* dst, float value, size_t n);
void orc_copy(const float* src, float* dst, size_t n);

/* Normalization (normalization.cc). */
void orc_layer_norm_fwd(const float* x, const float* gamma, const float* beta,
                        float* y, float* mean, float* rstd, size_t rows,
                        size_t cols);
void orc_layer_norm_bwd(const float* dy, const float* x, const float* gamma,
                        const float* mean, const float* rstd, float* dx,
                        size_t rows, size_t cols);
void orc_rms_norm_fwd(const float* x, const float* gamma, float* y,
                      float* rstd, size_t rows, size_t cols);
void orc_rms_norm_bwd(const float* dy, const float* x, const float* gamma,
                      const float* rstd, float* dx, size_t rows, size_t cols);

/* Transformer family (attention.cc). */
void orc_rope_fwd(const float* x, float* y, size_t B, size_t S, size_t H,
                  size_t d, float base);
void orc_rope_bwd(const float* dy, float* dx, size_t B, size_t S, size_t H,
                  size_t d, float base);
void orc_attn_fwd(const float* q, const float* k, const float* v, float* o,
                  float* probs, size_t B, size_t S, size_t H, size_t d);
void orc_attn_dp(const float* dout, const float* v, float* dp, size_t B,
                 size_t S, size_t H, size_t d);
void orc_attn_dv(const float* probs, const float* dout, float* dv, size_t B,
                 size_t S, size_t H, size_t d);
void orc_softmax_rows_bwd(const float* probs, const float* dp, float* ds,
                          size_t rows, size_t cols);
void orc_attn_dq(const float* ds, const float* k, float* dq, size_t B,
                 size_t S, size_t H, size_t d);
void orc_attn_dk(const float* ds, const float* q, float* dk, size_t B,
                 size_t S, size_t H, size_t d);

/* Losses (loss.cc). */
void orc_softmax_xent_fwd(const float* logits, const int32_t* labels,
                          float* loss, float* probs, size_t N, size_t C);
void orc_softmax_xent_bwd(const float* probs, const int32_t* labels,
                          const float* seed, float* dlogits, size_t N,
                          size_t C);
void orc_mse_fwd(const float* pred, const float* target, float* loss,
                 size_t n);
void orc_mse_bwd(const float* pred, const float* target, const float* seed,
                 float* dpred, size_t n);
void orc_kl_distill_fwd(const float* s_logits, const float* t_logits,
                        float* loss, float* p_s, float* p_t, size_t N,
                        size_t C, float T);
void orc_kl_distill_bwd(const float* p_s, const float* p_t, const float* seed,
                        float* dlogits, size_t N, size_t C, float T);

/* Optimizers (optimizer.cc). */
void orc_clip_norm(float* g, size_t n, float max_norm);
void orc_sgd_step(float* p, const float* g, size_t n, float lr, float wd);
void orc_adamw_step(float* p, const float* g, float* m, float* v, size_t n,
                    float lr, float beta1, float beta2, float eps, float wd,
                    uint64_t step);

/* Engine pieces (update_engine.cc). */
void orc_counter_randn(uint64_t seed, uint64_t count, float* out);
float orc_effective_lr(float lr, uint32_t schedule, uint64_t warmup_steps,
                       uint64_t default_steps, float min_lr_factor,
                       uint64_t step);
/* ExecuteRange restated over a decoded program of 64-byte instruction words
 * (`count` words at `program`). `lr` is EffectiveLr() for this step. */
void orc_execute(const void* program, size_t count, uint8_t* arena,
                 const uint8_t* rodata, float lr, float beta1, float beta2,
                 float eps, float weight_decay, uint64_t step);

#ifdef __cplusplus
}
#endif

#endif /* SEEML_ORACLE_H_ */
