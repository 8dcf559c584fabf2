// The quantizer surface the LeVo conversion tool calls, on device memory:
// ggml_quantize_chunk / ggml_row_size (tools/levo-quantize.cpp:386-388),
// padded_input_columns (src/levo-quantization.h:120-125), write_tensor's
// widen -> pad -> quantize chunk (tools/levo-quantize.cpp:355-388), the
// dequantizers and the F16 row converters (:358, :369), and the decode
// mat-vec of a Q8_0 matrix (ggml_mul_mat on the quantized LeLM / Flow
// weights, src/levo-quantization.h:96-118). Q8_0 and Q4_0 blocks are ggml's
// byte layouts. Errors are std::invalid_argument.
#pragma once

#include "levo-hip-device.h"

#include <cstddef>
#include <cstdint>

namespace levo::hip {

// Bytes of one row of n_per_row values (ggml_row_size).
std::size_t row_size(levo_hip_type type, int64_t n_per_row);

// Columns after zero-padding a row to whole blocks of `type`.
int64_t padded_input_columns(int64_t columns, levo_hip_type type);

// ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row, imatrix) with
// src and dst in device memory: quantizes rows [start / n_per_row, + nrows)
// and returns nrows * row_size(type, n_per_row).
std::size_t quantize_chunk(levo_hip_type type, const float * src, void * dst, int64_t start, int64_t nrows,
                           int64_t n_per_row, const float * imatrix = nullptr, stream_t stream = nullptr);

// write_tensor's quantized branch in one pass: nrows rows of src_cols values
// (F32, or F16 widened exactly) at src_row_stride elements, zero-padded to
// dst_cols and quantized. Returns the bytes written.
std::size_t quantize_rows(levo_hip_type type, const void * src, levo_hip_type src_type, int64_t src_cols,
                          int64_t src_row_stride, void * dst, int64_t nrows, int64_t dst_cols,
                          stream_t stream = nullptr);

// ggml's to_float for Q8_0 / Q4_0 (k a multiple of 32) and Q4_K / Q5_K / Q6_K
// (k a multiple of 256, src 16-byte aligned).
void dequantize_row(levo_hip_type type, const void * src, float * dst, int64_t k, stream_t stream = nullptr);

// ggml_mul_mat(W, x) for a Q8_0 weight at decode, as ggml's CPU backend
// computes it: x [n_vec][k] F32 is quantized to Q8_0 (ggml's vec_dot_type for
// Q8_0) into x_blocks (n_vec * row_size(Q8_0, k) bytes, 16-byte aligned), then
// y [n_vec][rows] = sum over blocks of sumi * (d_w * d_x). weight is
// [rows][k / 32] block_q8_0, 16-byte aligned; every pointer is device memory.
// For further matrices with the same input, mul_mat_q8_0_quantized reuses
// x_blocks. k a multiple of 32, 1 <= n_vec <= 8.
void mul_mat_q8_0(const void * weight, const float * x, void * x_blocks, float * y, int64_t rows, int64_t k,
                  int64_t n_vec, stream_t stream = nullptr);
void mul_mat_q8_0_quantized(const void * weight, const void * x_blocks, float * y, int64_t rows, int64_t k,
                            int64_t n_vec, stream_t stream = nullptr);

// Up to four Q8_0 matrices that read the same F32 input x [n_vec][k] (a
// layer's q / k / v, or gate / up) in one launch, the input quantized inside
// it: each y equals mul_mat_q8_0's for that matrix, bit for bit. Needs
// n_vec * k / 32 <= 256 and x 16-byte aligned; quantize larger inputs with
// mul_mat_q8_0 and reuse the blocks.
struct q8_0_matrix {
    const void * weight;  // [rows][k / 32] block_q8_0, 16-byte aligned
    float * y;            // [n_vec][rows]
    int64_t rows;
};
void mul_mat_q8_0_shared_input(const q8_0_matrix * mats, int n_mats, const float * x, int64_t k, int64_t n_vec,
                               stream_t stream = nullptr);

// The same mat-vecs on a Q8_0 matrix rearranged once when the model is
// loaded (repack_q8_0: packed holds the same rows * k / 32 * 34 bytes, each
// row's quants split in block halves, the scales after all rows; 16-byte
// aligned, not overlapping weight). The input goes through x_columns
// (q8_0_columns_size(n_vec, k) bytes, 16-byte aligned): the Q8_0
// quantization of x in the form the mat-vec keeps on chip. Each y equals
// mul_mat_q8_0's on the original blocks, bit for bit; the launch that reads
// the weights is 15-25 % shorter at LeLM's matrices.
void repack_q8_0(const void * weight, void * packed, int64_t rows, int64_t k, stream_t stream = nullptr);
std::size_t q8_0_columns_size(int64_t n_vec, int64_t k);
void mul_mat_q8_0_packed(const void * packed, const float * x, void * x_columns, float * y, int64_t rows,
                         int64_t k, int64_t n_vec, stream_t stream = nullptr);
void mul_mat_q8_0_packed_quantized(const void * packed, const void * x_columns, float * y, int64_t rows,
                                   int64_t k, int64_t n_vec, stream_t stream = nullptr);
// mul_mat_q8_0_shared_input on packed matrices (q8_0_matrix.weight from
// repack_q8_0).
void mul_mat_q8_0_packed_shared_input(const q8_0_matrix * mats, int n_mats, const float * x, int64_t k,
                                      int64_t n_vec, stream_t stream = nullptr);

// ggml_mul_mat(W, x) for a Q4_K / Q5_K / Q6_K weight at decode (the Q4_K_M,
// Q5_K_M and Q6_K profiles' matrices, src/levo-quantization.h:47-55, 96-118),
// as ggml's CPU backend computes it: x [n_vec][k] F32 is quantized to Q8_K
// (the K-quants' vec_dot_type) into x_blocks (n_vec * row_size(Q8_K, k)
// bytes, 4-byte aligned), then y [n_vec][rows] = ggml_vec_dot_q*_K_q8_K per
// row. weight is [rows][k / 256] blocks, 16-byte aligned; k a multiple of 256
// (padded_input_columns), 1 <= n_vec <= 8. mul_mat_kquant_quantized reuses
// x_blocks for further matrices with the same input.
void mul_mat_kquant(levo_hip_type type, const void * weight, const float * x, void * x_blocks, float * y,
                    int64_t rows, int64_t k, int64_t n_vec, stream_t stream = nullptr);
void mul_mat_kquant_quantized(levo_hip_type type, const void * weight, const void * x_blocks, float * y,
                              int64_t rows, int64_t k, int64_t n_vec, stream_t stream = nullptr);

// Up to four K-quant matrices, of any of Q4_K / Q5_K / Q6_K, that read the same
// F32 input x [n_vec][k] (a layer's q / k / v or gate / up under the Q4_K_M
// and Q5_K_M profiles, which mix in Q6_K matrices) in one launch, the input
// quantized to Q8_K inside it: each y equals mul_mat_kquant's for that matrix,
// bit for bit, when the matrices have equal row counts. Needs n_vec * k <=
// 4096 and x 16-byte aligned; quantize larger inputs with mul_mat_kquant and
// pass the blocks to mul_mat_kquant_quantized.
struct kquant_matrix {
    levo_hip_type type;
    const void * weight;  // [rows][k / 256] blocks, 16-byte aligned
    float * y;            // [n_vec][rows]
    int64_t rows;
};
void mul_mat_kquant_shared_input(const kquant_matrix * mats, int n_mats, const float * x, int64_t k, int64_t n_vec,
                                 stream_t stream = nullptr);

void fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n, stream_t stream = nullptr);
void fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n, stream_t stream = nullptr);

} // namespace levo::hip
