/* mx_oracle.h -- TEST INFRASTRUCTURE ONLY: declarations of the C restatement
 * in mx_oracle.c (the checker of tests/, smoke() and bench.py's CPU
 * baseline).  Not part of the product. */
#ifndef MX_ORACLE_H
#define MX_ORACLE_H
#include <stdint.h>

#define ORC_POOL_SUM 0
#define ORC_POOL_MEAN 1
#define ORC_FP32 0
#define ORC_FP16 1
#define ORC_INT8 2
#define ORC_INT4 3
#define ORC_INT2 4
#define ORC_FP8 6

float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
uint16_t orc_float_to_bf16(float f);
float orc_hfp8_to_float(uint8_t v, int32_t ebits, int32_t ebias);
uint8_t orc_float_to_hfp8(float x, int32_t ebits, int32_t ebias, float max_pos);

void orc_tbe_forward_f32(const float* W, const int64_t* w_off, const int32_t* D_off, int32_t T,
                         int64_t B, const int64_t* indices, const int64_t* offsets,
                         int32_t pooling, const float* iw, float* out, int64_t total_D);

int64_t orc_nbit_row_bytes(int32_t ty, int32_t D, int32_t row_align);

int orc_nbit_forward(const uint8_t* W, const int64_t* w_off, const uint8_t* tys,
                     const int32_t* D_off, int32_t T, int64_t B, const int64_t* indices,
                     const int64_t* offsets, int32_t pooling, const float* iw, int32_t row_align,
                     int32_t out_kind, void* out, int64_t total_D, int32_t fp8_ebits,
                     int32_t fp8_ebias);

int orc_transpose(const int64_t* hsc, int32_t T, int64_t B, int32_t nb, int32_t bits,
                  const int64_t* indices, const int64_t* offsets, int64_t N, int64_t* linear,
                  int64_t* sorted, int32_t* infos, int64_t* run, int32_t* run_lengths,
                  int64_t* num_runs, int32_t* cum);

int orc_backward_rowwise_adagrad(float* W, const int64_t* w_off, const int32_t* D_off,
                                 int32_t T, int64_t B, const int64_t* hsc, int32_t bits,
                                 const int64_t* indices, const int64_t* offsets, int64_t N,
                                 int32_t pooling, const float* iw, const float* grad,
                                 int64_t total_D, float* m1, const int64_t* m1_off, float lr,
                                 float eps, float wd, int32_t wd_mode, int32_t nb);
void orc_grad_indice_weights(const float* grad, int64_t total_D, const float* W,
                             const int64_t* w_off, const int32_t* D_off, int32_t T, int64_t B,
                             const int64_t* indices, const int64_t* offsets, int32_t pooling,
                             const int32_t* frg, float* giw);
int64_t orc_bounds_check(const int64_t* rows, int32_t T, int64_t B, int64_t* indices,
                         int64_t* offsets, int64_t N, int32_t mode);
int orc_nbit_forward_nobag(const uint8_t* W, const int64_t* w_off, const uint8_t* tys,
                           int32_t D, int32_t T, int64_t B, const int64_t* indices,
                           const int64_t* offsets, int32_t row_align, int32_t out_kind,
                           void* out, int32_t fp8_ebits, int32_t fp8_ebias);
int orc_backward_rowwise_adagrad_nobag(float* W, const int64_t* w_off, int32_t D, int32_t T,
                                       int64_t B, const int64_t* hsc, int32_t bits,
                                       const int64_t* indices, const int64_t* offsets, int64_t N,
                                       const float* grad, float* m1, const int64_t* m1_off,
                                       float lr, float eps, float wd, int32_t wd_mode,
                                       int32_t nb);
void orc_quantize_8bit(const float* x, int64_t rows, int64_t D, uint8_t* out);
void orc_dequantize_8bit(const uint8_t* in, int64_t rows, int64_t D, float* out);
void orc_quantize_nbit(const float* x, int64_t rows, int64_t D, int32_t bits, uint8_t* out);
void orc_dequantize_nbit(const uint8_t* in, int64_t rows, int64_t D, int32_t bits, float* out);
#endif
