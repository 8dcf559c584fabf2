// levo::hip op drop-ins on device tensor views: SnakeBeta (the reference KAT of
// tests/test-audio-ops.cpp:113-221 and the validation of
// src/levo-audio-ops.cpp:10-30, 129-141), the fused residual norms and the
// quantizer surface (tests/test-quantization.cpp:32-81), each also against
// the oracle at a LeVo shape.
#include "check.h"
#include "levo-hip-audio-ops.h"
#include "levo-hip-norms.h"
#include "levo-hip-quantize.h"
#include "levo_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <iostream>
#include <vector>

using namespace levo::hip;

namespace {

template <typename T>
struct device_vec {
    explicit device_vec(const std::vector<T> & host) : buf(host.size()), size(host.size()) {
        buf.upload(host.data(), host.size(), nullptr);
        synchronize(nullptr);
    }
    explicit device_vec(std::size_t n) : buf(n), size(n) {}
    std::vector<T> get() const {
        std::vector<T> out(size);
        buf.download(out.data(), size, nullptr);
        synchronize(nullptr);
        return out;
    }
    T * data() { return buf.data(); }
    device_buffer<T> buf;
    std::size_t size;
};

std::vector<float> gaussian(std::size_t n, uint64_t seed, float scale = 1.0F, float shift = 0.0F) {
    std::vector<float> v(n);
    lo_gaussian_noise(v.data(), static_cast<int64_t>(n), seed);
    for (auto & x : v) x = x * scale + shift;
    return v;
}

std::vector<uint16_t> to_f16(const std::vector<float> & v) {
    std::vector<uint16_t> h(v.size());
    lo_fp32_to_fp16_row(v.data(), h.data(), static_cast<int64_t>(v.size()));
    return h;
}

float rel_err(const std::vector<float> & got, const std::vector<float> & want) {
    float worst = 0.0F;
    for (std::size_t i = 0; i < got.size(); ++i) {
        worst = std::max(worst, std::fabs(got[i] - want[i]) / std::max(std::fabs(want[i]), 1.0F));
    }
    return worst;
}

int32_t f16_order(uint16_t h) { return (h & 0x8000) ? -static_cast<int32_t>(h & 0x7fff) : static_cast<int32_t>(h); }

int max_f16_ulp(const std::vector<uint16_t> & a, const std::vector<uint16_t> & b) {
    int worst = 0;
    for (std::size_t i = 0; i < a.size(); ++i) worst = std::max(worst, std::abs(f16_order(a[i]) - f16_order(b[i])));
    return worst;
}

void snake_reference_kat() {
    const std::vector<float> x = {-1.0F, 0.0F, 1.0F, -0.5F, 0.5F, 1.5F};
    const std::vector<float> a = {std::log(2.0F), std::log(0.5F)};
    const std::vector<float> b = {std::log(1.5F), std::log(0.75F)};
    std::vector<float> expected;
    for (std::size_t c = 0; c < 2; ++c) {
        const float alpha = std::exp(a[c]);
        const float beta = std::exp(b[c]) + 1.0e-9F;
        for (std::size_t t = 0; t < 3; ++t) {
            const float v = x[c * 3 + t];
            const float s = std::sin(v * alpha);
            expected.push_back(v + s * s / beta);
        }
    }
    device_vec<float> dx(x), da(a), db(b), dy(std::size_t{6});
    device_vec<uint16_t> ha(to_f16(a)), hb(to_f16(b));
    const tensor_view in = make_tensor_view(dx.data(), LEVO_HIP_TYPE_F32, 3, 2, 1);
    const tensor_view out = make_tensor_view(dy.data(), LEVO_HIP_TYPE_F32, 3, 2, 1);
    const tensor_view alpha = make_tensor_view(da.data(), LEVO_HIP_TYPE_F32, 1, 2, 1);
    const tensor_view beta = make_tensor_view(db.data(), LEVO_HIP_TYPE_F32, 1, 2, 1);
    detail::snake_beta(&in, &alpha, &beta, &out);
    std::vector<float> y = dy.get();
    for (std::size_t i = 0; i < 6; ++i) CHECK(std::fabs(y[i] - expected[i]) <= 1.0e-6F);
    const tensor_view alpha16 = make_tensor_view(ha.data(), LEVO_HIP_TYPE_F16, 1, 2, 1);
    const tensor_view beta16 = make_tensor_view(hb.data(), LEVO_HIP_TYPE_F16, 1, 2, 1);
    detail::snake_beta(&in, &alpha16, &beta16, &out);
    y = dy.get();
    for (std::size_t i = 0; i < 6; ++i) CHECK(std::fabs(y[i] - expected[i]) <= 2.0e-3F);
    // Mixed parameter types widen the F16 one exactly.
    detail::snake_beta(&in, &alpha, &beta16, &out);
    y = dy.get();
    for (std::size_t i = 0; i < 6; ++i) CHECK(std::fabs(y[i] - expected[i]) <= 2.0e-3F);

    // Validation messages.
    tensor_view bad = in;
    bad.type = LEVO_HIP_TYPE_F16;
    expect_throw<std::invalid_argument>("LeVo audio graph: SnakeBeta input is null",
                                        [&] { detail::snake_beta(nullptr, &alpha, &beta, &out); });
    expect_throw<std::invalid_argument>("LeVo audio graph: SnakeBeta input must be F32",
                                        [&] { detail::snake_beta(&bad, &alpha, &beta, &out); });
    tensor_view q = alpha;
    q.type = LEVO_HIP_TYPE_Q8_0;
    expect_throw<std::invalid_argument>("LeVo audio graph: SnakeBeta alpha_log must be F32 or F16",
                                        [&] { detail::snake_beta(&in, &q, &beta, &out); });
    expect_throw<std::invalid_argument>("LeVo audio graph: SnakeBeta beta_log is null",
                                        [&] { detail::snake_beta(&in, &alpha, nullptr, &out); });
    tensor_view wide = alpha;
    wide.ne[0] = 2;
    expect_throw<std::invalid_argument>("LeVo audio graph: SnakeBeta parameters must have shape [1, channels, 1]",
                                        [&] { detail::snake_beta(&in, &wide, &beta, &out); });
}

// Two batches of a [T=2016, C=512] activation with padded rows, in place.
void snake_parity() {
    const int64_t T = 2016, C = 512, pitch = 2020, B = 2;
    const std::vector<float> x = gaussian(static_cast<std::size_t>(pitch * C * B), 5, 2.0F);
    const std::vector<float> a = gaussian(static_cast<std::size_t>(C), 6, 0.3F);
    const std::vector<float> b = gaussian(static_cast<std::size_t>(C), 7, 0.3F);
    device_vec<float> dx(x), da(a), db(b);
    tensor_view in = make_tensor_view(dx.data(), LEVO_HIP_TYPE_F32, T, C, B);
    in.nb[1] = static_cast<std::size_t>(pitch) * 4;
    in.nb[2] = in.nb[1] * static_cast<std::size_t>(C);
    in.nb[3] = in.nb[2] * static_cast<std::size_t>(B);
    const tensor_view alpha = make_tensor_view(da.data(), LEVO_HIP_TYPE_F32, 1, C, 1);
    const tensor_view beta = make_tensor_view(db.data(), LEVO_HIP_TYPE_F32, 1, C, 1);
    detail::snake_beta(&in, &alpha, &beta, &in);
    const std::vector<float> got = dx.get();
    std::vector<float> packed(static_cast<std::size_t>(T * C)), want(static_cast<std::size_t>(T * C)), g(want.size());
    for (int64_t bt = 0; bt < B; ++bt) {
        for (int64_t c = 0; c < C; ++c) {
            std::copy_n(x.begin() + (bt * C + c) * pitch, T, packed.begin() + c * T);
            std::copy_n(got.begin() + (bt * C + c) * pitch, T, g.begin() + c * T);
        }
        lo_snake_beta_f32(packed.data(), a.data(), b.data(), want.data(), C, T, 4);
        CHECK(rel_err(g, want) <= 1.0e-5F);
        for (int64_t c = 0; c < C; ++c) {  // the row padding is untouched
            for (int64_t t = T; t < pitch; ++t) {
                const std::size_t i = static_cast<std::size_t>((bt * C + c) * pitch + t);
                CHECK(got[i] == x[i]);
            }
        }
    }
}

void norm_parity() {
    const int64_t D = 2048, R = 756;
    const std::size_t n = static_cast<std::size_t>(D * R);
    const std::vector<uint16_t> x = to_f16(gaussian(n, 21)), d = to_f16(gaussian(n, 22));
    const std::vector<uint16_t> w = to_f16(gaussian(static_cast<std::size_t>(D), 23, 0.02F, 1.0F));
    const std::vector<uint16_t> bias = to_f16(gaussian(static_cast<std::size_t>(D), 24, 0.02F));
    device_vec<uint16_t> dx(x), dd(d), dw(w), db(bias), dh(n), dy(n);
    const tensor_view vx = make_tensor_view(dx.data(), LEVO_HIP_TYPE_F16, D, R);
    const tensor_view vd = make_tensor_view(dd.data(), LEVO_HIP_TYPE_F16, D, R);
    const tensor_view vh = make_tensor_view(dh.data(), LEVO_HIP_TYPE_F16, D, R);
    const tensor_view vy = make_tensor_view(dy.data(), LEVO_HIP_TYPE_F16, D, R);
    const tensor_view vw = make_tensor_view(dw.data(), LEVO_HIP_TYPE_F16, D);
    const tensor_view vb = make_tensor_view(db.data(), LEVO_HIP_TYPE_F16, D);
    std::vector<uint16_t> wh(n), wy(n);

    residual_rms_norm(&vx, &vd, &vw, 1.0e-6F, &vh, &vy);
    lo_residual_rms_norm_f16(x.data(), d.data(), w.data(), wh.data(), wy.data(), R, D, 1.0e-6F, 4);
    CHECK(dh.get() == wh);
    CHECK(max_f16_ulp(dy.get(), wy) <= 1);

    residual_layer_norm(&vx, &vd, &vw, &vb, 1.0e-6F, &vh, &vy);
    lo_residual_layer_norm_f16(x.data(), d.data(), w.data(), bias.data(), wh.data(), wy.data(), R, D, 1.0e-6F, 4);
    CHECK(dh.get() == wh);
    CHECK(max_f16_ulp(dy.get(), wy) <= 1);

    // F32 tower, no residual.
    const std::vector<float> xf = gaussian(n, 25), wf = gaussian(static_cast<std::size_t>(D), 26, 0.02F, 1.0F);
    device_vec<float> fx(xf), fw(wf), fy(n);
    const tensor_view vfx = make_tensor_view(fx.data(), LEVO_HIP_TYPE_F32, D, R);
    const tensor_view vfy = make_tensor_view(fy.data(), LEVO_HIP_TYPE_F32, D, R);
    const tensor_view vfw = make_tensor_view(fw.data(), LEVO_HIP_TYPE_F32, D);
    residual_rms_norm(&vfx, nullptr, &vfw, 1.0e-5F, nullptr, &vfy);
    std::vector<float> want(n);
    lo_residual_rms_norm_f32(xf.data(), nullptr, wf.data(), nullptr, want.data(), R, D, 1.0e-5F, 4);
    CHECK(rel_err(fy.get(), want) <= 1.0e-5F);

    expect_throw<std::invalid_argument>("LeVo HIP norm: activation tensors must share one type",
                                        [&] { residual_rms_norm(&vx, &vfx, &vw, 1.0e-6F, nullptr, &vy); });
    expect_throw<std::invalid_argument>("LeVo HIP norm: weight must have shape [dim]", [&] {
        const tensor_view short_w = make_tensor_view(dw.data(), LEVO_HIP_TYPE_F16, D - 1);
        residual_rms_norm(&vx, nullptr, &short_w, 1.0e-6F, nullptr, &vy);
    });
}

// The Flow estimator's block boundary through the tensor-view wrapper: gate /
// scale / shift as ggml_view_2d chunks 2 / 4 / 3 of a [6 * dim, batch] time
// modulation (rows 6 * dim floats apart) plus a block table
// (src/levo-flow-estimator.cpp:95-104, 221-233).
void modulated_norm_parity() {
    const int64_t D = 2200, F = 100, B = 2;
    const std::size_t n = static_cast<std::size_t>(D * F * B);
    const std::vector<float> x = gaussian(n, 61), d = gaussian(n, 62);
    const std::vector<float> g = gaussian(static_cast<std::size_t>(D), 63, 0.02F, 1.0F);
    const std::vector<float> b = gaussian(static_cast<std::size_t>(D), 64, 0.02F);
    const std::vector<float> tm = gaussian(static_cast<std::size_t>(6 * D * B), 65, 0.3F);
    const std::vector<float> table = gaussian(static_cast<std::size_t>(6 * D), 66, 0.3F);
    device_vec<float> dx(x), dd(d), dg(g), db(b), dtm(tm), dtab(table), dh(n), dy(n);
    const tensor_view vx = make_tensor_view(dx.data(), LEVO_HIP_TYPE_F32, D, F, B);
    const tensor_view vd = make_tensor_view(dd.data(), LEVO_HIP_TYPE_F32, D, F, B);
    const tensor_view vh = make_tensor_view(dh.data(), LEVO_HIP_TYPE_F32, D, F, B);
    const tensor_view vy = make_tensor_view(dy.data(), LEVO_HIP_TYPE_F32, D, F, B);
    const tensor_view vg = make_tensor_view(dg.data(), LEVO_HIP_TYPE_F32, D);
    const tensor_view vb = make_tensor_view(db.data(), LEVO_HIP_TYPE_F32, D);
    tensor_view chunk[6], learned[6];
    for (int k = 0; k < 6; ++k) {
        chunk[k] = make_tensor_view(dtm.data() + k * D, LEVO_HIP_TYPE_F32, D, B);
        chunk[k].nb[1] = static_cast<std::size_t>(6 * D) * sizeof(float);  // ggml_view_2d of the modulation
        chunk[k].nb[2] = chunk[k].nb[3] = chunk[k].nb[1] * static_cast<std::size_t>(B);
        learned[k] = make_tensor_view(dtab.data() + k * D, LEVO_HIP_TYPE_F32, D);
    }
    residual_layer_norm_modulated(&vx, &vd, {&chunk[2], &learned[2]}, &vg, &vb, {&chunk[4], &learned[4]},
                                  {&chunk[3], &learned[3]}, 1.0e-5F, &vh, &vy);
    const lo_batch_vector gate{tm.data() + 2 * D, 6 * D, table.data() + 2 * D};
    const lo_batch_vector scale{tm.data() + 4 * D, 6 * D, table.data() + 4 * D};
    const lo_batch_vector shift{tm.data() + 3 * D, 6 * D, table.data() + 3 * D};
    std::vector<float> wh(n), wy(n);
    lo_residual_layer_norm_modulated_f32(x.data(), d.data(), &gate, g.data(), b.data(), &scale, &shift, wh.data(),
                                         wy.data(), F * B, F, D, 1.0e-5F);
    CHECK(dh.get() == wh);
    CHECK(rel_err(dy.get(), wy) <= 1.0e-5F);

    expect_throw<std::invalid_argument>("LeVo HIP norm: scale must have shape [dim, batch]", [&] {
        const tensor_view one = make_tensor_view(dtm.data(), LEVO_HIP_TYPE_F32, D, 1);
        residual_layer_norm_modulated(&vx, &vd, {}, &vg, &vb, {&one, nullptr}, {&chunk[3], nullptr}, 1.0e-5F,
                                      nullptr, &vy);
    });
    expect_throw<std::invalid_argument>("LeVo HIP norm: scale and shift come together", [&] {
        residual_layer_norm_modulated(&vx, &vd, {}, &vg, &vb, {&chunk[4], nullptr}, {}, 1.0e-5F, nullptr, &vy);
    });
}

void quantize_surface() {
    // tests/test-quantization.cpp:45-51: a 4 x 32 matrix with six live columns.
    std::vector<float> original(32 * 4, 0.0F);
    for (int row = 0; row < 4; ++row) {
        for (int column = 0; column < 6; ++column) {
            original[static_cast<std::size_t>(row * 32 + column)] = 0.03125F * static_cast<float>((row + 1) * (column + 1));
        }
    }
    CHECK(row_size(LEVO_HIP_TYPE_Q8_0, 32) == 34 && row_size(LEVO_HIP_TYPE_Q4_0, 32) == 18);
    CHECK(padded_input_columns(2200, LEVO_HIP_TYPE_Q8_0) == 2208);
    CHECK(padded_input_columns(4400, LEVO_HIP_TYPE_Q4_0) == 4416);
    CHECK(padded_input_columns(2200, LEVO_HIP_TYPE_F16) == 2200);
    device_vec<float> src(original), deq(std::size_t{128});
    device_vec<uint8_t> q(std::size_t{34 * 4});
    CHECK(quantize_chunk(LEVO_HIP_TYPE_Q8_0, src.data(), q.data(), 0, 4, 32, nullptr) == 34 * 4);
    std::vector<uint8_t> want(34 * 4);
    CHECK(lo_quantize_chunk(LEVO_HIP_TYPE_Q8_0, original.data(), want.data(), 0, 4, 32) == want.size());
    CHECK(q.get() == want);
    dequantize_row(LEVO_HIP_TYPE_Q8_0, q.data(), deq.data(), 128);
    const std::vector<float> back = deq.get();
    const float input[6] = {0.25F, -0.5F, 0.75F, -1.0F, 1.25F, -1.5F};
    for (int row = 0; row < 4; ++row) {
        float expected = 0.0F, actual = 0.0F;
        for (int column = 0; column < 6; ++column) {
            expected += original[static_cast<std::size_t>(row * 32 + column)] * input[column];
            actual += back[static_cast<std::size_t>(row * 32 + column)] * input[column];
        }
        CHECK(std::fabs(actual - expected) < 0.015F);
    }
    expect_throw<std::invalid_argument>(nullptr, [&] {
        (void) quantize_chunk(LEVO_HIP_TYPE_Q8_0, src.data(), q.data(), 0, 4, 31, nullptr);
    });

    // write_tensor's chunk path: F16 [rows, 2200] -> zero-padded 2208-column Q4_0 / Q8_0.
    const int64_t rows = 64, cols = 2200, padded = 2208;
    const std::vector<uint16_t> h = to_f16(gaussian(static_cast<std::size_t>(rows * cols), 31, 0.02F));
    device_vec<uint16_t> dh(h);
    for (levo_hip_type t : {LEVO_HIP_TYPE_Q8_0, LEVO_HIP_TYPE_Q4_0}) {
        const std::size_t bytes = row_size(t, padded) * static_cast<std::size_t>(rows);
        device_vec<uint8_t> dq(bytes);
        CHECK(quantize_rows(t, dh.data(), LEVO_HIP_TYPE_F16, cols, cols, dq.data(), rows, padded) == bytes);
        std::vector<uint8_t> w(bytes);
        CHECK(lo_quantize_f16_rows_padded(t, h.data(), rows, cols, padded, w.data()) == bytes);
        CHECK(dq.get() == w);
    }

    // F16 row converters round-trip against the oracle.
    const std::vector<float> f = gaussian(4099, 41, 100.0F);
    device_vec<float> df(f), dback(std::size_t{4099});
    device_vec<uint16_t> dhalf(std::size_t{4099});
    fp32_to_fp16_row(df.data(), dhalf.data(), 4099);
    fp16_to_fp32_row(dhalf.data(), dback.data(), 4099);
    const std::vector<uint16_t> want_h = to_f16(f);
    CHECK(dhalf.get() == want_h);
    std::vector<float> want_back(4099);
    lo_fp16_to_fp32_row(want_h.data(), want_back.data(), 4099);
    const std::vector<float> got_back = dback.get();
    CHECK(bit_equal(got_back.data(), want_back.data(), 4099));
}

// The Q8_0 decode mat-vec against the oracle's ggml CPU restatement: the
// CFG pair at LeLM's ffn_down shape (1536 x 8960) within F32 rounding, and an
// integer-valued case (d = 1 blocks) exactly.
void mul_mat_surface() {
    const int64_t rows = 1536, k = 8960, n_vec = 2;
    std::vector<float> w = gaussian(static_cast<std::size_t>(rows * k), 51, 0.02F);
    const std::vector<float> x = gaussian(static_cast<std::size_t>(n_vec * k), 52, 1.0F);
    std::vector<uint8_t> wb(row_size(LEVO_HIP_TYPE_Q8_0, k) * static_cast<std::size_t>(rows));
    CHECK(lo_quantize_chunk(LEVO_HIP_TYPE_Q8_0, w.data(), wb.data(), 0, rows, k) == wb.size());
    std::vector<float> want(static_cast<std::size_t>(n_vec * rows));
    lo_mul_mat_q8_0(wb.data(), x.data(), want.data(), rows, k, n_vec);
    device_vec<uint8_t> dw(wb), dxb(row_size(LEVO_HIP_TYPE_Q8_0, k) * static_cast<std::size_t>(n_vec) + 16);
    device_vec<float> dx(x), dy(static_cast<std::size_t>(n_vec * rows));
    mul_mat_q8_0(dw.data(), dx.data(), dxb.data(), dy.data(), rows, k, n_vec);
    const std::vector<float> got = dy.get();
    for (std::size_t i = 0; i < got.size(); ++i) {
        CHECK(std::fabs(got[i] - want[i]) <= 1e-5F * std::max(1.0F, std::fabs(want[i])));
    }

    const int64_t ir = 40, ik = 640;
    std::vector<float> iw(static_cast<std::size_t>(ir * ik)), ix(static_cast<std::size_t>(2 * ik));
    for (std::size_t i = 0; i < iw.size(); ++i) iw[i] = i % 32 == 0 ? 127.0F : static_cast<float>(static_cast<int>(i * 7919 % 255) - 127);
    for (std::size_t i = 0; i < ix.size(); ++i) ix[i] = i % 32 == 3 ? -127.0F : static_cast<float>(static_cast<int>(i * 104729 % 255) - 127);
    std::vector<uint8_t> iwb(row_size(LEVO_HIP_TYPE_Q8_0, ik) * static_cast<std::size_t>(ir));
    CHECK(lo_quantize_chunk(LEVO_HIP_TYPE_Q8_0, iw.data(), iwb.data(), 0, ir, ik) == iwb.size());
    device_vec<uint8_t> diw(iwb), dixb(row_size(LEVO_HIP_TYPE_Q8_0, ik) * 2 + 16);
    device_vec<float> dix(ix), diy(static_cast<std::size_t>(2 * ir));
    mul_mat_q8_0(diw.data(), dix.data(), dixb.data(), diy.data(), ir, ik, 2);
    const std::vector<float> igot = diy.get();
    for (int64_t v = 0; v < 2; ++v) {
        for (int64_t r = 0; r < ir; ++r) {
            int64_t exact = 0;
            for (int64_t c = 0; c < ik; ++c) {
                exact += static_cast<int64_t>(iw[static_cast<std::size_t>(r * ik + c)]) *
                         static_cast<int64_t>(ix[static_cast<std::size_t>(v * ik + c)]);
            }
            CHECK(igot[static_cast<std::size_t>(v * ir + r)] == static_cast<float>(exact));
        }
    }
    expect_throw<std::invalid_argument>("multiple of 32", [&] {
        mul_mat_q8_0_quantized(dw.data(), dxb.data(), dy.data(), rows, 100, n_vec);
    });

    // two matrices sharing the F32 input in one launch (the second is the
    // first 7 rows of the same blocks): the same exact integers
    device_vec<float> dy40(static_cast<std::size_t>(2 * ir)), dy7(2 * 7);
    const q8_0_matrix mats[2] = {{diw.data(), dy40.data(), ir}, {diw.data(), dy7.data(), 7}};
    mul_mat_q8_0_shared_input(mats, 2, dix.data(), ik, 2);
    CHECK(bit_equal(dy40.get().data(), igot.data(), igot.size()));
    const std::vector<float> got7 = dy7.get();
    for (int64_t v = 0; v < 2; ++v) {
        CHECK(bit_equal(got7.data() + v * 7, igot.data() + v * ir, 7));
    }
    expect_throw<std::invalid_argument>("<= 256 blocks", [&] {
        const q8_0_matrix big[1] = {{dw.data(), dy.data(), rows}};
        mul_mat_q8_0_shared_input(big, 1, dx.data(), k, n_vec);
    });

    // the packed matrices: the same y, bit for bit
    device_vec<uint8_t> dp(wb.size()), dxc(q8_0_columns_size(n_vec, k));
    device_vec<float> dyp(static_cast<std::size_t>(n_vec * rows));
    repack_q8_0(dw.data(), dp.data(), rows, k);
    mul_mat_q8_0_packed(dp.data(), dx.data(), dxc.data(), dyp.data(), rows, k, n_vec);
    CHECK(bit_equal(dyp.get().data(), got.data(), got.size()));
    device_vec<uint8_t> dip(iwb.size());
    device_vec<float> dyp40(static_cast<std::size_t>(2 * ir));
    repack_q8_0(diw.data(), dip.data(), ir, ik);
    const q8_0_matrix pmats[1] = {{dip.data(), dyp40.data(), ir}};
    mul_mat_q8_0_packed_shared_input(pmats, 1, dix.data(), ik, 2);
    CHECK(bit_equal(dyp40.get().data(), igot.data(), igot.size()));
    expect_throw<std::invalid_argument>("must not overlap", [&] { repack_q8_0(dw.data(), dw.data(), rows, k); });
}

// K-quant decode path: padded_input_columns for 256-value blocks
// (src/levo-quantization.h:120-130), dequantize_row bit-exact on random
// blocks, and mul_mat_kquant exact on integer-valued blocks (d = dmin = 1,
// Q8_K d = 1), all against the oracle.
void kquant_surface() {
    CHECK(padded_input_columns(2200, LEVO_HIP_TYPE_Q4_K) == 2304);
    CHECK(padded_input_columns(4400, LEVO_HIP_TYPE_Q6_K) == 4608);
    CHECK(padded_input_columns(2304, LEVO_HIP_TYPE_Q5_K) == 2304);
    const uint16_t one = 0x3C00, small = 0x1400;  // F16 1.0 and 2^-10
    for (levo_hip_type type : {LEVO_HIP_TYPE_Q4_K, LEVO_HIP_TYPE_Q5_K, LEVO_HIP_TYPE_Q6_K}) {
        const std::size_t bb = row_size(type, 256);
        const int64_t rows = 24, k = 1536, nb = rows * k / 256;
        std::vector<uint8_t> wb(bb * static_cast<std::size_t>(nb));
        uint64_t state = 0x9E3779B97F4A7C15ULL + static_cast<uint64_t>(type);
        for (auto & b : wb) {
            state = state * 6364136223846793005ULL + 1442695040888963407ULL;
            b = static_cast<uint8_t>(state >> 56);
        }
        for (int64_t i = 0; i < nb; ++i) {  // finite scales
            uint8_t * blk = wb.data() + static_cast<std::size_t>(i) * bb;
            if (type == LEVO_HIP_TYPE_Q6_K) {
                std::memcpy(blk + 208, &small, 2);
            } else {
                std::memcpy(blk, &small, 2);
                std::memcpy(blk + 2, &small, 2);
            }
        }
        std::vector<float> want(static_cast<std::size_t>(rows * k));
        lo_dequantize_row_kquant(type, wb.data(), want.data(), rows * k);
        device_vec<uint8_t> dw(wb);
        device_vec<float> dq(static_cast<std::size_t>(rows * k));
        dequantize_row(type, dw.data(), dq.data(), rows * k);
        const std::vector<float> got = dq.get();
        CHECK(bit_equal(got.data(), want.data(), got.size()));

        for (int64_t i = 0; i < nb; ++i) {  // integer-valued blocks
            uint8_t * blk = wb.data() + static_cast<std::size_t>(i) * bb;
            if (type == LEVO_HIP_TYPE_Q6_K) {
                std::memcpy(blk + 208, &one, 2);
            } else {
                std::memcpy(blk, &one, 2);
                std::memcpy(blk + 2, &one, 2);
            }
        }
        std::vector<float> x(static_cast<std::size_t>(2 * k));
        for (std::size_t i = 0; i < x.size(); ++i) {
            x[i] = i % 256 == 0 ? -127.0F : static_cast<float>(static_cast<int>(i * 104729 % 255) - 127);
        }
        std::vector<float> ywant(static_cast<std::size_t>(2 * rows));
        lo_mul_mat_kquant(type, wb.data(), x.data(), ywant.data(), rows, k, 2);
        device_vec<uint8_t> dwi(wb), dxb(row_size(LEVO_HIP_TYPE_Q8_K, k) * 2);
        device_vec<float> dx(x), dy(static_cast<std::size_t>(2 * rows));
        mul_mat_kquant(type, dwi.data(), dx.data(), dxb.data(), dy.data(), rows, k, 2);
        const std::vector<float> ygot = dy.get();
        CHECK(bit_equal(ygot.data(), ywant.data(), ygot.size()));
    }
    expect_throw<std::invalid_argument>("multiple of 256", [&] {
        (void) row_size(LEVO_HIP_TYPE_Q4_K, 300);
    });
}

} // namespace

int main() {
    try {
        snake_reference_kat();
        snake_parity();
        norm_parity();
        modulated_norm_parity();
        quantize_surface();
        mul_mat_surface();
        kquant_surface();
    } catch (const std::exception & e) {
        std::cerr << "unexpected exception: " << e.what() << '\n';
        return 1;
    }
    std::cout << "hip ops ok\n";
    return 0;
}
