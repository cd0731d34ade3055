// k_hbm_roof.hip -- measurement kernels for the practical HBM roof of the
// access patterns the path's bandwidth-bound kernels use.  Built into its
// own library (libfg_hbm_roof.so), loaded only by bench.py; nothing in the
// product calls it.  Each kernel streams fp32 data with 16-byte
// non-temporal accesses, one 4 KiB chunk per thread block pass (256 threads
// x 16 bytes), in the layout that measured fastest for a plain copy.
//
//   read:   sum every element of src (1 stream read; one float per block
//           written so the loads cannot be dropped)
//   copy:   dst = src (1 read, 1 write)
//   s3r3w:  o1 = a * b, o2 = o1 + c, o3 = o2 (3 read, 3 write: the stream
//           count of the elementwise program tanh(a * b + c))
//   s4r3w:  p, m, v updated from p, g, m, v with multiply-adds (4 read,
//           3 write: the stream count of Adam)
//   rows:   y = x - rowmax(x) over rows of C <= 32768 floats, with the row
//           structure of the softmax + CE kernel: one workgroup reads its
//           whole row into registers (16-byte buffer loads), reduces it
//           across the workgroup, then writes it -- 512 threads x 16 float4,
//           or 1024 threads x 8 float4 held to 64 VGPRs (two workgroups per
//           CU) as the softmax kernel runs rows of more than 16384 columns
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;

__device__ __forceinline__ f32x4 ld(const f32x4 *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st(f32x4 *p, f32x4 v) { __builtin_nontemporal_store(v, p); }

__global__ __launch_bounds__(kThreads) void read_k(const f32x4 *src, uint64_t nq, float *out) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < nq;
         i += (uint64_t)gridDim.x * kThreads)
        s += ld(src + i);
    float t = s[0] + s[1] + s[2] + s[3];
    for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o);
    __shared__ float w[kThreads / 64];
    if ((threadIdx.x & 63) == 0) w[threadIdx.x >> 6] = t;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = w[0] + w[1] + w[2] + w[3];
}

__global__ __launch_bounds__(kThreads) void copy_k(const f32x4 *src, f32x4 *dst, uint64_t nq) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < nq;
         i += (uint64_t)gridDim.x * kThreads)
        st(dst + i, ld(src + i));
}

__global__ __launch_bounds__(kThreads) void s3r3w_k(const f32x4 *a, const f32x4 *b,
                                                    const f32x4 *c, f32x4 *o1, f32x4 *o2,
                                                    f32x4 *o3, uint64_t nq) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < nq;
         i += (uint64_t)gridDim.x * kThreads) {
        const f32x4 x = ld(a + i) * ld(b + i);
        const f32x4 y = x + ld(c + i);
        st(o1 + i, x);
        st(o2 + i, y);
        st(o3 + i, y);
    }
}

__global__ __launch_bounds__(kThreads) void s4r3w_k(f32x4 *p, const f32x4 *g, f32x4 *m,
                                                    f32x4 *v, uint64_t nq) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < nq;
         i += (uint64_t)gridDim.x * kThreads) {
        const f32x4 gg = ld(g + i);
        const f32x4 mm = 0.9f * ld(m + i) + 0.1f * gg;
        const f32x4 vv = 0.999f * ld(v + i) + 0.001f * gg * gg;
        st(m + i, mm);
        st(v + i, vv);
        st(p + i, ld(p + i) - 1e-3f * mm);
    }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufWord3 = 0x00020000;  // buffer descriptor word 3 for gfx9 targets
constexpr int kBufNT = 2;              // cache-policy bits: non-temporal

// Chunk k (NT float4) of a row: a descriptor whose range ends at the row's
// end, so lanes past it read zero and have their stores dropped.
template <int NT>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float *row, int C, int k) {
    const int skip = k * NT * 16;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(row) + skip / 4, (short)0,
                                             max(C * 4 - skip, 0), kBufWord3);
}

template <int NV, int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT >= 1024 ? 8 : 1)))
void rows_k(const float *x, float *y, int C) {
    constexpr int NW = NT / 64;
    __shared__ float sm[NW];
    const float *xr = x + (size_t)blockIdx.x * C;
    float *yr = y + (size_t)blockIdx.x * C;
    const int off = (int)threadIdx.x * 16;
    f32x4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i)
        v[i] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(row_rsrc<NT>(xr, C, i), off, 0, kBufNT));
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const bool in = (int)threadIdx.x + NT * i < C / 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) m = in ? fmaxf(m, v[i][e]) : m;
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = m;
    __syncthreads();
    m = sm[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) m = fmaxf(m, sm[k]);
#pragma unroll
    for (int i = 0; i < NV; ++i)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[i] - m),
                                               row_rsrc<NT>(yr, C, i), off, 0, kBufNT);
}

// One block per 4 KiB chunk up to the 32-bit work-item limit; the loops
// cover the rest.
unsigned blocks_for(uint64_t nq) {
    uint64_t b = (nq + kThreads - 1) / kThreads;
    const uint64_t cap = (uint64_t(1) << 32) / kThreads / 2;
    return (unsigned)(b < cap ? b : cap);
}

int status() { return hipGetLastError() == hipSuccess ? 0 : 1; }

}  // namespace

// n: fp32 elements per stream, a multiple of 4; pointers 16-byte aligned;
// `out` of the read probe holds one float per block (blocks_for(n / 4)).
extern "C" __attribute__((visibility("default"))) int fg_roof_blocks(uint64_t n) {
    return (int)blocks_for(n / 4);
}
extern "C" __attribute__((visibility("default"))) int fg_roof_read(void *stream, const float *src,
                                                                   uint64_t n, float *out) {
    read_k<<<blocks_for(n / 4), kThreads, 0, (hipStream_t)stream>>>(
        reinterpret_cast<const f32x4 *>(src), n / 4, out);
    return status();
}
extern "C" __attribute__((visibility("default"))) int fg_roof_copy(void *stream, const float *src,
                                                                   float *dst, uint64_t n) {
    copy_k<<<blocks_for(n / 4), kThreads, 0, (hipStream_t)stream>>>(
        reinterpret_cast<const f32x4 *>(src), reinterpret_cast<f32x4 *>(dst), n / 4);
    return status();
}
extern "C" __attribute__((visibility("default"))) int fg_roof_s3r3w(void *stream, const float *a,
                                                                    const float *b, const float *c,
                                                                    float *o1, float *o2, float *o3,
                                                                    uint64_t n) {
    s3r3w_k<<<blocks_for(n / 4), kThreads, 0, (hipStream_t)stream>>>(
        reinterpret_cast<const f32x4 *>(a), reinterpret_cast<const f32x4 *>(b),
        reinterpret_cast<const f32x4 *>(c), reinterpret_cast<f32x4 *>(o1),
        reinterpret_cast<f32x4 *>(o2), reinterpret_cast<f32x4 *>(o3), n / 4);
    return status();
}
extern "C" __attribute__((visibility("default"))) int fg_roof_s4r3w(void *stream, float *p,
                                                                    const float *g, float *m,
                                                                    float *v, uint64_t n) {
    s4r3w_k<<<blocks_for(n / 4), kThreads, 0, (hipStream_t)stream>>>(
        reinterpret_cast<f32x4 *>(p), reinterpret_cast<const f32x4 *>(g),
        reinterpret_cast<f32x4 *>(m), reinterpret_cast<f32x4 *>(v), n / 4);
    return status();
}
// R rows of C floats (C % 4 == 0, 0 < C <= 32768, rows 16-byte aligned and
// contiguous); wide: the 1024-thread form.
extern "C" __attribute__((visibility("default"))) int fg_roof_rows(void *stream, const float *x,
                                                                   float *y, int R, int C,
                                                                   int wide) {
    if (R <= 0 || C <= 0 || C % 4 != 0 || C > 32768) return 1;
    if (wide)
        rows_k<8, 1024><<<R, 1024, 0, (hipStream_t)stream>>>(x, y, C);
    else
        rows_k<16, 512><<<R, 512, 0, (hipStream_t)stream>>>(x, y, C);
    return status();
}
