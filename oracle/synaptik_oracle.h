/* CPU restatement of the reference's fp32 MLP training path: test infrastructure only
 * (see synaptik_oracle.c). Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline. */
#ifndef SYNAPTIK_ORACLE_H
#define SYNAPTIK_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
void shko_matmul_f32(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                     int64_t lda, int64_t ldb, int64_t ldc, int trans_a, int trans_b);
float shko_exact_sum(const float* x, int64_t n, int64_t stride);
float shko_exact_mean(const float* x, int64_t n, int64_t stride);
float shko_exact_quotient(float value, int64_t count);
float shko_max(const float* x, int64_t n, int64_t stride);
void shko_colsum(const float* X, float* out, int64_t R, int64_t N, int64_t ldx);
void shko_activation(int act, const float* x, float* y, int64_t n);
void shko_activation_grad(int act, const float* g, const float* y, float* dx, int64_t n);
void shko_linear_forward(const float* X, const float* W, const float* b, float* Y, int64_t B,
                         int64_t in, int64_t out, int act);
void shko_softmax_rows(const float* X, float* Y, int64_t R, int64_t C, int log_softmax);
void shko_logsumexp_rows(const float* X, float* out, int64_t R, int64_t C);
void shko_softmax_grad_rows(const float* Y, const float* G, float* DX, int64_t R, int64_t C);
void shko_logsumexp_grad_rows(const float* X, const float* lse, const float* g, float* DX,
                              int64_t R, int64_t C);
float shko_mse_mean(const float* p, const float* t, int64_t n);
float shko_mse_mean_exact(const float* p, const float* t, int64_t n);
float shko_mse_sum(const float* p, const float* t, int64_t n);
void shko_mse_grad(const float* p, const float* t, float* grad, int64_t n, float g, int sum);
int shko_index_ce_mean(const float* logits, const int64_t* target, int64_t R, int64_t C,
                       int has_ignore, int64_t ignore, float* loss);
void shko_index_ce_grad(const float* logits, const int64_t* target, float* grad, int64_t R,
                        int64_t C, int has_ignore, int64_t ignore, float g);
int shko_sgd_stage(const float* p, const float* g, const float* m, float* p_out, float* m_out,
                   int64_t n, float lr, float momentum, float dampening, float weight_decay,
                   int nesterov, int has_momentum_slot, int64_t completed_steps);
int shko_adam_apply(const float* p, const float* m_new, const float* v_new, float* p_out,
                    int64_t n, float lr, float b1, float b2, float eps, float decay,
                    int decoupled, int64_t completed_steps);
int shko_adam_stage(const float* p, const float* g, const float* m, const float* v, float* p_out,
                    float* m_out, float* v_out, int64_t n, float lr, float b1, float b2, float eps,
                    float decay, int decoupled, int64_t completed_steps);
int shko_canonical_bytes(const uint8_t* src, uint64_t src_bytes, int width, int boolean,
                         int rank, const int64_t* dims, const int64_t* strides, int64_t offset,
                         uint8_t* dst);
#ifdef __cplusplus
}
#endif
#endif
