// Plain streaming kernels that measure what one launch can move at a given
// byte count and read / write mix on this GPU: the ceiling an op of that size
// and mix is compared with. Reads and writes are dwordx4, coalesced, each
// vector touched once; nothing is computed. Not part of the kernel library:
// the benchmark loads this file's own shared object.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Thread i handles vectors i, i + stride, ... (VPT of them): it reads
// src[v] for v < n_read and writes dst[v] for v < n_write (the value read, or
// zero past n_read). A read-only launch (n_write = 0) keeps its loads alive
// with a store that never happens for finite data.
template <int VPT>
__global__ __launch_bounds__(256) void stream_kernel(const f32x4 * __restrict__ src, f32x4 * __restrict__ dst,
                                                     int64_t n_read, int64_t n_write, int64_t stride) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    f32x4 v[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t i = base + k * stride;
        v[k] = i < n_read ? __builtin_nontemporal_load(src + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    float sink = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t i = base + k * stride;
        if (i < n_write) __builtin_nontemporal_store(v[k], dst + i);
        else sink += v[k].x;
    }
    if (sink == __builtin_inff() && n_write > 0) dst[0] = v[0];
}

}  // namespace

// Moves read_bytes from src and write_bytes to dst (both multiples of 16,
// buffers 16-byte aligned) with `vpt` vectors per thread (1, 2 or 4).
extern "C" int levo_bench_stream(const void * src, void * dst, int64_t read_bytes, int64_t write_bytes, int vpt,
                                 hipStream_t stream) {
    const int64_t nr = read_bytes / 16, nw = write_bytes / 16;
    const int64_t n = nr > nw ? nr : nw;
    if (n <= 0 || (vpt != 1 && vpt != 2 && vpt != 4)) return -1;
    const int64_t threads = (n + vpt - 1) / vpt;
    const int64_t blocks = (threads + 255) / 256;
    if (blocks >= (int64_t{1} << 31)) return -1;
    const int64_t stride = blocks * 256;
    const auto s = static_cast<const f32x4 *>(src);
    auto d = static_cast<f32x4 *>(dst);
    if (vpt == 1) stream_kernel<1><<<static_cast<uint32_t>(blocks), 256, 0, stream>>>(s, d, nr, nw, stride);
    else if (vpt == 2) stream_kernel<2><<<static_cast<uint32_t>(blocks), 256, 0, stream>>>(s, d, nr, nw, stride);
    else stream_kernel<4><<<static_cast<uint32_t>(blocks), 256, 0, stream>>>(s, d, nr, nw, stride);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
