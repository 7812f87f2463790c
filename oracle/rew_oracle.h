/* rew_oracle.h -- CPU restatement of rew's eager op semantics.
 * TEST INFRASTRUCTURE ONLY (see rew_oracle.c). */
#ifndef REW_ORACLE_H
#define REW_ORACLE_H

#include <stdint.h>

enum { ORC_F32 = 0, ORC_BF16 = 1 };
enum { ORC_ADD = 0, ORC_SUB, ORC_MUL, ORC_DIV, ORC_MAX, ORC_MIN, ORC_POW, ORC_REM, ORC_ATAN2 };
enum { ORC_NEG = 0, ORC_ABS, ORC_EXP, ORC_LOG, ORC_SQRT, ORC_RSQRT, ORC_TANH, ORC_LOGISTIC,
       ORC_SIN, ORC_COS, ORC_FLOOR, ORC_CEIL };
enum { ORC_RSUM = 0, ORC_RMAX, ORC_RMIN, ORC_RPROD };

void orc_threefry(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1, uint32_t out[2]);
void orc_split(uint32_t k0, uint32_t k1, int n, uint32_t* out);
void orc_fold_in(uint32_t k0, uint32_t k1, uint64_t data, uint32_t out[2]);
void orc_uniform_f32(uint32_t k0, uint32_t k1, int64_t n, float lo, float hi, float* out);
void orc_normal_f32(uint32_t k0, uint32_t k1, int64_t n, float mean, float sd, float* out);

int orc_num_threads(void);

uint16_t orc_bf16(float f);
float orc_bf16_f32(uint16_t h);
void orc_f32_to_bf16(const float* x, int64_t n, uint16_t* out);
void orc_bf16_to_f32(const uint16_t* x, int64_t n, float* out);

float orc_binary_scalar(int op, float a, float b);
void orc_binary_f32(int op, const float* a, const float* b, float* out, int64_t n);
float orc_unary_scalar(int op, float x);
void orc_unary_f32(int op, const float* a, float* out, int64_t n);

void orc_reduce_f32(int op, const float* x, int rank, const int64_t* shape, int ndims,
                    const int64_t* dims, float* out);
void orc_dot_general(int dt, const void* a, int ra, const int64_t* sa, const void* b, int rb,
                     const int64_t* sb, int nbatch, const int64_t* lb, const int64_t* rbd,
                     int ncon, const int64_t* lc, const int64_t* rc, void* out);
void orc_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
              int round_bf16);

void orc_softmax_rows(const float* x, int64_t rows, int64_t cols, float* out);
void orc_rmsnorm_rows(const float* x, const float* gamma, int64_t rows, int64_t cols, float eps,
                      float* out);
void orc_layernorm_rows(const float* x, const float* gamma, const float* beta, int64_t rows,
                        int64_t cols, float eps, float* out);
void orc_rope(const float* x, const float* cos_t, const float* sin_t, int64_t outer, int64_t S,
              int64_t D, int64_t offset, float* out);
void orc_sdpa(const float* q, const float* k, const float* v, int64_t B, int64_t H,
              int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, int causal, float scale, int mixed,
              float* out);
void orc_argmax_rows(const float* x, int64_t rows, int64_t cols, int32_t* out);
void orc_topk_rows(const float* x, int64_t rows, int64_t cols, int64_t k, float* vals,
                   int32_t* idx);

#endif
