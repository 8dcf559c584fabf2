#include "levo-hip-quantize.h"

namespace levo::hip {

std::size_t row_size(levo_hip_type type, int64_t n_per_row) {
    return static_cast<std::size_t>(check_status(levo_hip_row_size(type, n_per_row)));
}

int64_t padded_input_columns(int64_t columns, levo_hip_type type) {
    int64_t block = 0;  // ggml_blck_size of the quantized types
    if (type == LEVO_HIP_TYPE_Q8_0 || type == LEVO_HIP_TYPE_Q4_0) block = 32;
    if (type == LEVO_HIP_TYPE_Q4_K || type == LEVO_HIP_TYPE_Q5_K || type == LEVO_HIP_TYPE_Q6_K) block = 256;
    if (block == 0) return columns;
    if (columns <= 0) return columns;
    return (columns + block - 1) / block * block;
}

std::size_t quantize_chunk(levo_hip_type type, const float * src, void * dst, int64_t start, int64_t nrows,
                           int64_t n_per_row, const float * imatrix, stream_t stream) {
    return static_cast<std::size_t>(
            check_status(levo_hip_quantize_chunk(type, src, dst, start, nrows, n_per_row, imatrix, stream)));
}

std::size_t quantize_rows(levo_hip_type type, const void * src, levo_hip_type src_type, int64_t src_cols,
                          int64_t src_row_stride, void * dst, int64_t nrows, int64_t dst_cols, stream_t stream) {
    return static_cast<std::size_t>(check_status(
            levo_hip_quantize_rows(type, src, src_type, src_cols, src_row_stride, dst, nrows, dst_cols, stream)));
}

void mul_mat_q8_0(const void * weight, const float * x, void * x_blocks, float * y, int64_t rows, int64_t k,
                  int64_t n_vec, stream_t stream) {
    if (rows == 0 || n_vec == 0) return;
    check_status(levo_hip_quantize_chunk(LEVO_HIP_TYPE_Q8_0, x, x_blocks, 0, n_vec, k, nullptr, stream));
    mul_mat_q8_0_quantized(weight, x_blocks, y, rows, k, n_vec, stream);
}

void mul_mat_q8_0_quantized(const void * weight, const void * x_blocks, float * y, int64_t rows, int64_t k,
                            int64_t n_vec, stream_t stream) {
    check_status(levo_hip_mul_mat_q8_0(weight, x_blocks, y, rows, rows, k, n_vec, stream));
}

void mul_mat_q8_0_shared_input(const q8_0_matrix * mats, int n_mats, const float * x, int64_t k, int64_t n_vec,
                               stream_t stream) {
    levo_hip_mat_q8_0 m[4] = {};
    const int n = n_mats < 0 ? 0 : n_mats;
    for (int i = 0; i < n && i < 4; ++i) m[i] = levo_hip_mat_q8_0{mats[i].weight, mats[i].y, mats[i].rows, mats[i].rows};
    check_status(levo_hip_mul_mat_q8_0_multi(m, n_mats, nullptr, x, k, k, n_vec, stream));
}

void repack_q8_0(const void * weight, void * packed, int64_t rows, int64_t k, stream_t stream) {
    check_status(levo_hip_repack_q8_0(weight, packed, rows, k, stream));
}

std::size_t q8_0_columns_size(int64_t n_vec, int64_t k) {
    if (n_vec < 0 || k < 0 || k % 32 != 0) throw std::invalid_argument("q8_0_columns_size: bad size");
    return static_cast<std::size_t>(n_vec) * static_cast<std::size_t>(k / 32) * 36;
}

void mul_mat_q8_0_packed(const void * packed, const float * x, void * x_columns, float * y, int64_t rows, int64_t k,
                         int64_t n_vec, stream_t stream) {
    if (rows == 0 || n_vec == 0) return;
    check_status(levo_hip_quantize_q8_0_columns(x, k, x_columns, n_vec, k, stream));
    mul_mat_q8_0_packed_quantized(packed, x_columns, y, rows, k, n_vec, stream);
}

void mul_mat_q8_0_packed_quantized(const void * packed, const void * x_columns, float * y, int64_t rows, int64_t k,
                                   int64_t n_vec, stream_t stream) {
    check_status(levo_hip_mul_mat_q8_0_packed(packed, x_columns, y, rows, rows, k, n_vec, stream));
}

void mul_mat_q8_0_packed_shared_input(const q8_0_matrix * mats, int n_mats, const float * x, int64_t k,
                                      int64_t n_vec, stream_t stream) {
    levo_hip_mat_q8_0 m[4] = {};
    const int n = n_mats < 0 ? 0 : n_mats;
    for (int i = 0; i < n && i < 4; ++i) m[i] = levo_hip_mat_q8_0{mats[i].weight, mats[i].y, mats[i].rows, mats[i].rows};
    check_status(levo_hip_mul_mat_q8_0_packed_multi(m, n_mats, nullptr, x, k, k, n_vec, stream));
}

void mul_mat_kquant(levo_hip_type type, const void * weight, const float * x, void * x_blocks, float * y,
                    int64_t rows, int64_t k, int64_t n_vec, stream_t stream) {
    if (rows == 0 || n_vec == 0) return;
    check_status(levo_hip_quantize_q8_K(x, x_blocks, n_vec * k, stream));
    mul_mat_kquant_quantized(type, weight, x_blocks, y, rows, k, n_vec, stream);
}

void mul_mat_kquant_quantized(levo_hip_type type, const void * weight, const void * x_blocks, float * y,
                              int64_t rows, int64_t k, int64_t n_vec, stream_t stream) {
    check_status(levo_hip_mul_mat_kquant(type, weight, x_blocks, y, rows, rows, k, n_vec, stream));
}

void mul_mat_kquant_shared_input(const kquant_matrix * mats, int n_mats, const float * x, int64_t k, int64_t n_vec,
                                 stream_t stream) {
    levo_hip_mat_kquant m[4] = {};
    const int n = n_mats < 0 ? 0 : n_mats;
    for (int i = 0; i < n && i < 4; ++i) {
        m[i] = levo_hip_mat_kquant{mats[i].type, mats[i].weight, mats[i].y, mats[i].rows, mats[i].rows};
    }
    check_status(levo_hip_mul_mat_kquant_multi(m, n_mats, nullptr, x, k, k, n_vec, stream));
}

void dequantize_row(levo_hip_type type, const void * src, float * dst, int64_t k, stream_t stream) {
    check_status(levo_hip_dequantize(type, src, dst, LEVO_HIP_TYPE_F32, k, stream));
}

void fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n, stream_t stream) {
    check_status(levo_hip_fp32_to_fp16_row(x, y, n, stream));
}

void fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n, stream_t stream) {
    check_status(levo_hip_fp16_to_fp32_row(x, y, n, stream));
}

} // namespace levo::hip
