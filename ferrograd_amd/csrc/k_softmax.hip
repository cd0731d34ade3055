// k_softmax.hip -- row softmax, fused softmax + cross-entropy (forward and
// backward), softmax backward, for gfx950.
//
// Reference: the softmax node (crates/ferrograd-nn/src/op/softmax.rs:112-446)
// makes three passes over each row with 256-thread LDS tree reductions
// (read x twice, write e, read-modify-write e), the CE loss kernel
// (crates/fused_gpu/src/dispatch/backend/kernel/loss.rs:12-165 with
// basic_loss.rs:91-133) is a separate launch writing a full [R,C] loss
// buffer, and its gradient is then pushed through the softmax Jacobian a
// second time (defect).
//
// Here one workgroup owns one row.  The fast path keeps the whole row in
// registers (NV float4 per thread; 256 threads, or 1024 for rows of more
// than 16384 columns: up to 32768 columns), so the logits are read from HBM
// exactly once and dlogits written exactly once: 8*C bytes per row, the
// minimum.  Reductions are wavefront shuffles (64 lanes) followed by one LDS
// exchange across the waves.  Rows too long for registers, or not 16-byte
// aligned, use a two-pass streaming kernel with an online max/sum.
//
// Long rows (up to 32768 columns): 1024 threads with 8 float4 each, held
// to 64 VGPRs so that two workgroups share a CU, read and written with
// buffer instructions: the 8192 x 32000 CE at 5.76-5.84 TB/s (median of 30)
// against 5.70-5.75 for 512 threads with 16 float4 (two or three
// workgroups per CU) and 4.5-4.8 for 1024 threads at 4 waves per SIMD (one
// workgroup per CU: its reductions and exponentials leave the CU's memory
// idle).  Earlier, on the 512-thread kernel: 363.5 us (5.77 TB/s) against
// 372.5 us for 256 threads with 32 float4 and plain global accesses; measured
// and dropped: rotating each row's chunk order by the row index (366.9 us),
// holding the 512-thread kernel to 80 VGPRs for a sixth wave per SIMD (it
// then spills: 381 us), 256 threads with buffer instructions (377 us).  For
// scale: a flat copy of the same bytes reaches 6.5-6.6 TB/s, and copy kernels
// with this kernel's row structure (one workgroup reads a 128 KB row into
// registers, reduces it, writes it) 5.8 TB/s with 512 threads and 6.0 with
// 1024; capping each wave's loads in flight at 4, 8 or 12 of 16, walking the
// rows in another order, or a persistent workgroup that loads the next row
// while it finishes one leave them within 1-3 %.
#include <hip/hip_runtime.h>

#include <cmath>

#include "fg_half.h"
#include "fg_internal.h"
#include "fg_softmax_row.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kNT = 256;
constexpr int kWaves = kNT / 64;

using fg::smrow::argmax_combine;

// Block-wide (max, lowest index of max) over NW waves; every thread
// receives the result.
template <int NW = kWaves>
__device__ __forceinline__ void block_argmax(float &m, int &idx, float *sm, int *si) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float m2 = __shfl_xor(m, o);
        const int i2 = __shfl_xor(idx, o);
        argmax_combine(m, idx, m2, i2);
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sm[w] = m;
        si[w] = idx;
    }
    __syncthreads();
    m = sm[0];
    idx = si[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) argmax_combine(m, idx, sm[k], si[k]);
    __syncthreads();
}

template <int NW = kWaves>
__device__ __forceinline__ float block_sum(float s, float *sm) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sm[w] = s;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int k = 0; k < NW; ++k) t += sm[k];
    __syncthreads();
    return t;
}

// (max, sum of exp(x - max)) pairs for the streaming kernel.
__device__ __forceinline__ void ms_combine(float &m, float &s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) return;
    s = s * expf(m - mn) + s2 * expf(m2 - mn);
    m = mn;
}

__device__ __forceinline__ void block_ms(float &m, float &s, float *sm, float *ss) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float m2 = __shfl_xor(m, o);
        const float s2 = __shfl_xor(s, o);
        ms_combine(m, s, m2, s2);
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sm[w] = m;
        ss[w] = s;
    }
    __syncthreads();
    m = sm[0];
    s = ss[0];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) ms_combine(m, s, sm[k], ss[k]);
    __syncthreads();
}

// Row epilogue shared by the kernels: loss and argmax from thread 0.  xr
// is the row of logits of element type dt.
__device__ __forceinline__ void row_outputs(const void *xr, int dt, int C, const uint32_t *labels,
                                            int r, float m, float s, int am, float *row_loss,
                                            uint32_t *argmax) {
    if (threadIdx.x != 0) return;
    if (argmax) argmax[r] = (uint32_t)am;
    if (row_loss) {
        const uint32_t t = labels ? labels[r] : 0u;
        // A label outside [0, C) has no logit; report NaN rather than read.
        row_loss[r] =
            (t < (uint32_t)C) ? (m + logf(s)) - fg::load_as_f(xr, dt, t) : __builtin_nanf("");
    }
}

// Register-resident fast path with NT threads.  out (may be NULL) receives
//   labels ? scale*(p - onehot) : scale*p.
// Thread t holds the float4 chunks t + NT*i of the row (i < NV); argmax ties
// go to the lowest column (a row of -inf gives 0, as the CPU restatement's
// first-maximum scan does).  Rows are
// read and written with buffer instructions: each chunk gets a descriptor
// (uniform, in scalar registers) whose base is the chunk's start and whose
// size is what remains of the row, and every access takes the one 32-bit
// lane offset 16 * t.  The NV loads in flight then hold no 64-bit addresses
// in vector registers, and lanes past the row end read zero (replaced by
// -inf) and have their stores dropped by the descriptor's range check,
// which covers the vector offset (a raw buffer access does not range-check
// its scalar offset, so none is used).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufWord3 = 0x00020000;  // buffer descriptor word 3 for gfx9 targets
constexpr int kBufNT = 2;              // cache-policy bits: non-temporal

// A 1024-thread workgroup is held to 64 VGPRs (8 waves per SIMD), so that
// two rows share a CU and one's reductions and exponentials overlap the
// other's memory traffic.
template <int NV, int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT >= 1024 ? 8 : 1)))
void softmax_rows_v4(const float *__restrict__ x, int ldx,
                                                      const uint32_t *__restrict__ labels, int C,
                                                      float scale, float *__restrict__ row_loss,
                                                      float *__restrict__ out, int ldo,
                                                      uint32_t *__restrict__ argmax,
                                                      float *__restrict__ probs, int ldp) {
    constexpr int NW = NT / 64;
    __shared__ float sm[NW];
    __shared__ int si[NW];
    const int r = blockIdx.x;
    const float *xr = x + (size_t)r * ldx;
    const int C4 = C >> 2;
    const int lane_off = (int)threadIdx.x * 16;
    // Descriptor of chunk k of a row: base at the chunk, size = the row's
    // remaining bytes (0 past the end).
    auto rsrc = [&](const float *row, int k) {
        const int skip = k * NT * 16;
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(row) + skip / 4, (short)0,
                                                 max(C * 4 - skip, 0), kBufWord3);
    };
    f32x4 v[NV];
    float m = -INFINITY;
    int am = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rsrc(xr, i), lane_off, 0,
                                                              kBufNT);
        v[i] = __builtin_bit_cast(f32x4, w);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = (int)threadIdx.x + NT * i;
        if (j >= C4) v[i] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (v[i][e] > m || (v[i][e] == m && 4 * j + e < am)) {
                m = v[i][e];
                am = 4 * j + e;
            }
    }
    block_argmax<NW>(m, am, sm, si);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[i][e] = expf(v[i][e] - m);
            s += v[i][e];
        }
    }
    s = block_sum<NW>(s, sm);
    row_outputs(xr, fg::kF32, C, labels, r, m, s, am, row_loss, argmax);
    if (out) {
        const float inv = 1.0f / s;
        // The label's chunk and lane (none when unlabelled or out of range).
        const int t = labels ? (int)labels[r] : -1;
        const int jt = t >= 0 ? t >> 2 : -1, et = t & 3;
        const float *orow = out + (size_t)r * ldo;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = (int)threadIdx.x + NT * i;
            f32x4 d = v[i] * inv;
            if (j == jt) d[et] -= 1.0f;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, scale * d),
                                                   rsrc(orow, i), lane_off, 0, kBufNT);
        }
    }
    if (probs) {  // the softmax itself (the forward's output, when the loss writes it)
        const float inv = 1.0f / s;
        const float *prow = probs + (size_t)r * ldp;
#pragma unroll
        for (int i = 0; i < NV; ++i)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[i] * inv),
                                                   rsrc(prow, i), lane_off, 0, kBufNT);
    }
}

// Streaming path for any C, alignment and element type dt (x and out share
// it): pass 1 online (max, sum, argmax), pass 2 recomputes exp and writes,
// rounding to dt.
__global__ __launch_bounds__(kNT) void softmax_rows_stream(const void *__restrict__ x, int ldx,
                                                           const uint32_t *__restrict__ labels,
                                                           int C, float scale,
                                                           float *__restrict__ row_loss,
                                                           void *__restrict__ out, int ldo,
                                                           uint32_t *__restrict__ argmax, int dt,
                                                           void *__restrict__ probs, int ldp) {
    __shared__ float sm[kWaves], ss[kWaves];
    __shared__ int si[kWaves];
    const int r = blockIdx.x;
    const uint64_t xb = (uint64_t)r * ldx;
    float m = -INFINITY, s = 0.0f, am_m = -INFINITY;
    int am = 0x7fffffff;
    for (int c = threadIdx.x; c < C; c += kNT) {
        const float xv = fg::load_as_f(x, dt, xb + c);
        if (xv > am_m) {
            am_m = xv;
            am = c;
        }
        ms_combine(m, s, xv, 1.0f);
    }
    block_argmax(am_m, am, sm, si);
    block_ms(m, s, sm, ss);
    const size_t esz = dt == fg::kF32 ? 4 : 2;
    row_outputs(static_cast<const char *>(x) + xb * esz, dt, C, labels, r, m, s, am, row_loss,
                argmax);
    if (out || probs) {
        const float inv = 1.0f / s;
        const int t = labels ? (int)labels[r] : -1;
        const uint64_t ob = (uint64_t)r * ldo, pb = (uint64_t)r * ldp;
        for (int c = threadIdx.x; c < C; c += kNT) {
            const float p = expf(fg::load_as_f(x, dt, xb + c) - m) * inv;
            if (out) fg::store_from_f(out, dt, ob + c, scale * (c == t ? p - 1.0f : p));
            if (probs) fg::store_from_f(probs, dt, pb + c, p);
        }
    }
}

// Register-resident path for 16-bit rows (fp16 / bf16, 8-byte aligned,
// C % 4 == 0): NV groups of 4 elements per thread, read once, written once.
template <int NV>
__global__ __launch_bounds__(kNT) void softmax_rows_h4(const uint16_t *__restrict__ x, int ldx,
                                                       const uint32_t *__restrict__ labels, int C,
                                                       float scale, float *__restrict__ row_loss,
                                                       uint16_t *__restrict__ out, int ldo,
                                                       uint32_t *__restrict__ argmax, int dt,
                                                       uint16_t *__restrict__ probs, int ldp) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    __shared__ float sm[kWaves];
    __shared__ int si[kWaves];
    const int r = blockIdx.x;
    const uint16_t *xr = x + (size_t)r * ldx;
    const int C4 = C >> 2;
    f32x4 v[NV];
    float m = -INFINITY;
    int am = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = threadIdx.x + i * kNT;
        if (j < C4) {
            const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(xr) + j);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[i][e] = fg::h16_to_f(dt, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
        } else {
            v[i] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c0 = 4 * (threadIdx.x + i * kNT);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (v[i][e] > m) {
                m = v[i][e];
                am = c0 + e;
            }
    }
    block_argmax(m, am, sm, si);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[i][e] = expf(v[i][e] - m);
            s += v[i][e];
        }
    }
    s = block_sum(s, sm);
    row_outputs(xr, dt, C, labels, r, m, s, am, row_loss, argmax);
    if (out) {
        const float inv = 1.0f / s;
        const int t = labels ? (int)labels[r] : -1;
        uint16_t *orow = out + (size_t)r * ldo;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = threadIdx.x + i * kNT;
            if (j < C4) {
                uint16_t d[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float p = v[i][e] * inv;
                    d[e] = fg::f_to_h16(dt, scale * (4 * j + e == t ? p - 1.0f : p));
                }
                const u32x2 w = {(uint32_t)d[0] | ((uint32_t)d[1] << 16),
                                 (uint32_t)d[2] | ((uint32_t)d[3] << 16)};
                __builtin_nontemporal_store(w, reinterpret_cast<u32x2 *>(orow) + j);
            }
        }
    }
    if (probs) {
        const float inv = 1.0f / s;
        uint16_t *prow = probs + (size_t)r * ldp;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = threadIdx.x + i * kNT;
            if (j < C4) {
                uint16_t d[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) d[e] = fg::f_to_h16(dt, v[i][e] * inv);
                const u32x2 w = {(uint32_t)d[0] | ((uint32_t)d[1] << 16),
                                 (uint32_t)d[2] | ((uint32_t)d[3] << 16)};
                __builtin_nontemporal_store(w, reinterpret_cast<u32x2 *>(prow) + j);
            }
        }
    }
}

// Small problems in one workgroup (R <= kSmallRows, C <= kSmallCols): one
// wave per row (rows w, w + 16, ... for wave w of 16), a lane per column, so
// softmax + CE and the mean of the row losses take a single launch.  Max,
// argmax and the sum of exponentials are 64-lane shuffle trees; the mean sums
// each wave's rows in order (lane 0, double), then the waves in order.  The
// same outputs, conventions (argmax = first maximum, NaN loss for a label
// outside [0, C)) and element-type handling as the row kernels; `probs`
// receives the softmax itself.  A wave loads kSmallBatch rows (and labels)
// at once and takes the label's logit from the lane holding it, so c1's
// 64 x 10 loss is one memory round trip.
constexpr int kSmallCols = 64;
constexpr int kSmallRows = 1024;
constexpr int kSmallNT = 1024;
constexpr int kSmallWaves = kSmallNT / 64;
constexpr int kSmallBatch = 4;
bool small_case(int R, int C) { return C <= kSmallCols && R <= kSmallRows; }

template <int DT>
__device__ __forceinline__ float small_load(const void *p, uint64_t i) {
    if constexpr (DT == fg::kF32) return static_cast<const float *>(p)[i];
    else return fg::h16_to_f(DT, static_cast<const uint16_t *>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void small_store(void *p, uint64_t i, float v) {
    if constexpr (DT == fg::kF32) static_cast<float *>(p)[i] = v;
    else static_cast<uint16_t *>(p)[i] = fg::f_to_h16(DT, v);
}

template <int DT>
__global__ __launch_bounds__(kSmallNT) void softmax_ce_small(
    const void *__restrict__ x, int ldx, const uint32_t *__restrict__ labels, int R, int C,
    float scale, float *__restrict__ row_loss, void *__restrict__ out, int ldo,
    uint32_t *__restrict__ argmax, void *__restrict__ probs, int ldp, float *__restrict__ mean) {
    __shared__ double sh[kSmallWaves];
    const int c = threadIdx.x & 63, w = threadIdx.x >> 6;
    double acc = 0.0;  // this wave's row losses, in row order
    // kSmallBatch rows per pass: their loads are all issued before any use.
    for (int r0 = w; r0 < R; r0 += kSmallWaves * kSmallBatch) {
        float v[kSmallBatch];
        uint32_t t[kSmallBatch];
#pragma unroll
        for (int j = 0; j < kSmallBatch; ++j) {
            const int r = r0 + j * kSmallWaves;
            v[j] = (r < R && c < C) ? small_load<DT>(x, (uint64_t)r * ldx + c) : -INFINITY;
            t[j] = (r < R && labels) ? labels[r] : 0u;
        }
#pragma unroll
        for (int j = 0; j < kSmallBatch; ++j) {
            const int r = r0 + j * kSmallWaves;
            if (r >= R) break;
            float m = v[j];
            int am = c < C ? c : C;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1)
                argmax_combine(m, am, __shfl_xor(m, o), __shfl_xor(am, o));
            const float e = c < C ? expf(v[j] - m) : 0.0f;
            float s = e;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
            if (argmax && c == 0) argmax[r] = (uint32_t)am;
            if (row_loss || mean) {
                // The label's logit from the lane that holds it.
                const float xt = __shfl(v[j], (int)(t[j] & 63u));
                const float l = (t[j] < (uint32_t)C) ? (m + logf(s)) - xt : __builtin_nanf("");
                if (row_loss && c == 0) row_loss[r] = l;
                acc += (double)l;
            }
            if ((out || probs) && c < C) {
                const float pv = e * (1.0f / s);
                if (out)
                    small_store<DT>(out, (uint64_t)r * ldo + c,
                                    scale * (labels && (uint32_t)c == t[j] ? pv - 1.0f : pv));
                if (probs) small_store<DT>(probs, (uint64_t)r * ldp + c, pv);
            }
        }
    }
    if (!mean) return;
    if (c == 0) sh[w] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double tot = sh[0];
        for (int k = 1; k < kSmallWaves; ++k) tot += sh[k];
        mean[0] = (float)(tot / (double)R);
    }
}

// Heads of at most kTinyCols columns (c1's ten classes) in the same one
// workgroup: a row fits in one 16-lane row of a wave, so a wave takes four
// rows at once and reduces each inside its 16 lanes with four DPP moves
// (swap neighbours, swap pairs, half-row mirror, row mirror) -- register
// moves, where the wave-per-row kernel above chains 19 LDS-routed shuffles
// per row.  Each step combines a lane's value with another's by a
// commutative operation, so every lane of a row ends with the same max,
// argmax (first maximum) and sum, the sum always in the same order.  The
// label's logit is the row sum of (column == label ? logit : 0), exact.
// Row slot q (4 per wave, 64 in all) takes rows q, q + 64, ...; a wave
// loads kSmallBatch rows per slot at once; the mean adds each slot's rows
// in order (double), then the slots in order.  Outputs and conventions as
// softmax_ce_small.
constexpr int kTinyCols = fg::smrow::kCols;
constexpr int kTinySlots = kSmallNT / kTinyCols;
static_assert(kTinySlots == fg::smrow::kSlots, "row slots");
bool tiny_case(int R, int C) { return C <= kTinyCols && R <= kSmallRows; }

template <int DT>
__global__ __launch_bounds__(kSmallNT) void softmax_ce_tiny(
    const void *__restrict__ x, int ldx, const uint32_t *__restrict__ labels, int R, int C,
    float scale, float *__restrict__ row_loss, void *__restrict__ out, int ldo,
    uint32_t *__restrict__ argmax, void *__restrict__ probs, int ldp, float *__restrict__ mean) {
    __shared__ double sh[kTinySlots];
    const int lane = threadIdx.x & 63, c = lane & (kTinyCols - 1);
    const int q = lane / kTinyCols, w = threadIdx.x >> 6;
    const int slot = w * (64 / kTinyCols) + q;
    double acc = 0.0;  // this slot's row losses, in row order
    // The wave's first slot bounds the loop, so all 64 lanes run every pass
    // (the DPP moves read the other lanes of the row); rows past R compute
    // and store nothing.
    for (int b0 = w * (64 / kTinyCols); b0 < R; b0 += kTinySlots * kSmallBatch) {
        const int r0 = b0 + q;
        float v[kSmallBatch];
        uint32_t t[kSmallBatch];
#pragma unroll
        for (int j = 0; j < kSmallBatch; ++j) {
            const int r = r0 + j * kTinySlots;
            v[j] = (r < R && c < C) ? small_load<DT>(x, (uint64_t)r * ldx + c) : -INFINITY;
            t[j] = (r < R && labels) ? labels[r] : 0u;
        }
#pragma unroll
        for (int j = 0; j < kSmallBatch; ++j) {
            const int r = r0 + j * kTinySlots;
            const bool want_loss = row_loss || mean;
            const float l = fg::smrow::ce_row16<DT>(v[j], t[j], c, C, r, r < R, labels != nullptr,
                                                    scale, row_loss, out, ldo, argmax, probs, ldp,
                                                    want_loss);
            if (r < R && want_loss) acc += (double)l;
        }
    }
    if (!mean) return;
    if (c == 0) sh[slot] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double tot = sh[0];
        for (int k = 1; k < kTinySlots; ++k) tot += sh[k];
        mean[0] = (float)(tot / (double)R);
    }
}

// mean[0] = sum(vals[0..n)) / n in a fixed order (one block).
__global__ __launch_bounds__(1024) void mean_kernel(const float *__restrict__ vals, int n,
                                                    float *__restrict__ mean) {
    __shared__ double sh[1024];
    double acc = 0.0;
    for (int i = threadIdx.x; i < n; i += 1024) acc += (double)vals[i];
    sh[threadIdx.x] = acc;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) sh[threadIdx.x] += sh[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) mean[0] = n > 0 ? (float)(sh[0] / (double)n) : 0.0f;
}

// dx (=|+=) y * (dy - sum(dy*y)) per row (softmax.rs:448-688, all columns);
// y, dy, dx of element type dt, the result rounded to it once.
__global__ __launch_bounds__(kNT) void softmax_bwd_rows(const void *__restrict__ y,
                                                        const void *__restrict__ dy, int C,
                                                        void *__restrict__ dx, int accumulate,
                                                        int dt) {
    __shared__ float sm[kWaves];
    const uint64_t base = (uint64_t)blockIdx.x * C;
    float dot = 0.0f;
    for (int c = threadIdx.x; c < C; c += kNT)
        dot += fg::load_as_f(dy, dt, base + c) * fg::load_as_f(y, dt, base + c);
    dot = block_sum(dot, sm);
    for (int c = threadIdx.x; c < C; c += kNT) {
        const float g = fg::load_as_f(y, dt, base + c) * (fg::load_as_f(dy, dt, base + c) - dot);
        fg::store_from_f(dx, dt, base + c, accumulate ? fg::load_as_f(dx, dt, base + c) + g : g);
    }
}

// The row kernels for R rows of C; `probs` (may be NULL) receives the
// softmax.  With `mean` given and a small problem, the one-workgroup kernel
// also writes the mean loss and *mean_done is set; otherwise the caller
// reduces the row losses.
// The one-workgroup kernels (small_case): 16-lane rows for heads of at
// most kTinyCols columns, else a wave per row.
template <int DT>
void launch_small(hipStream_t st, const void *x, int ldx, const uint32_t *labels, int R, int C,
                  float scale, float *row_loss, void *out, int ldo, uint32_t *argmax, void *probs,
                  int ldp, float *mean) {
    if (tiny_case(R, C))
        softmax_ce_tiny<DT><<<1, kSmallNT, 0, st>>>(x, ldx, labels, R, C, scale, row_loss, out, ldo,
                                                   argmax, probs, ldp, mean);
    else
        softmax_ce_small<DT><<<1, kSmallNT, 0, st>>>(x, ldx, labels, R, C, scale, row_loss, out,
                                                    ldo, argmax, probs, ldp, mean);
}

int launch_rows(fg_ctx *ctx, int dt, const void *x, int ldx, const uint32_t *labels, int R, int C,
                float scale, float *row_loss, void *out, int ldo, uint32_t *argmax,
                void *probs = nullptr, int ldp = 0, float *mean = nullptr,
                bool *mean_done = nullptr) {
    hipStream_t st = ctx->stream;
    if (mean_done) *mean_done = false;
    if (small_case(R, C)) {
        if (dt == fg::kF32)
            launch_small<fg::kF32>(st, x, ldx, labels, R, C, scale, row_loss, out, ldo, argmax,
                                   probs, ldp, mean);
        else if (dt == fg::kBF16)
            launch_small<fg::kBF16>(st, x, ldx, labels, R, C, scale, row_loss, out, ldo, argmax,
                                    probs, ldp, mean);
        else
            launch_small<fg::kF16>(st, x, ldx, labels, R, C, scale, row_loss, out, ldo, argmax,
                                   probs, ldp, mean);
        FG_LAUNCH_CHECK("softmax_ce_small");
        if (mean_done) *mean_done = mean != nullptr;
        return FG_OK;
    }
    const unsigned align = dt == fg::kF32 ? 16u : 8u;
    const bool aligned = ((((uintptr_t)x) | ((uintptr_t)out) | ((uintptr_t)probs)) &
                          (align - 1)) == 0 &&
                         (C % 4 == 0) && (ldx % 4 == 0) && (!out || ldo % 4 == 0) &&
                         (!probs || ldp % 4 == 0);
    const int C4 = C / 4;
    dim3 grid(R), block(kNT);
    if (dt == fg::kF32) {
        const float *xf = static_cast<const float *>(x);
        float *of = static_cast<float *>(out);
#define FG_SM_LAUNCH(NV, NT)                                                               \
    softmax_rows_v4<NV, NT><<<grid, NT, 0, st>>>(xf, ldx, labels, C, scale, row_loss, of, ldo, \
                                                 argmax, static_cast<float *>(probs), ldp)
        if (aligned && C4 <= kNT * 1)
            FG_SM_LAUNCH(1, kNT);
        else if (aligned && C4 <= kNT * 2)
            FG_SM_LAUNCH(2, kNT);
        else if (aligned && C4 <= kNT * 4)
            FG_SM_LAUNCH(4, kNT);
        else if (aligned && C4 <= kNT * 8)
            FG_SM_LAUNCH(8, kNT);
        else if (aligned && C4 <= kNT * 16)
            FG_SM_LAUNCH(16, kNT);
        else if (aligned && C4 <= 4 * kNT * 8)
            FG_SM_LAUNCH(8, 4 * kNT);
        else
            softmax_rows_stream<<<grid, block, 0, st>>>(x, ldx, labels, C, scale, row_loss, out,
                                                        ldo, argmax, dt, probs, ldp);
#undef FG_SM_LAUNCH
    } else {
        const uint16_t *xh = static_cast<const uint16_t *>(x);
        uint16_t *oh = static_cast<uint16_t *>(out);
#define FG_SM_LAUNCH(NV)                                                                        \
    softmax_rows_h4<NV><<<grid, block, 0, st>>>(xh, ldx, labels, C, scale, row_loss, oh, ldo, \
                                                argmax, dt, static_cast<uint16_t *>(probs), ldp)
        if (aligned && C4 <= kNT * 1)
            FG_SM_LAUNCH(1);
        else if (aligned && C4 <= kNT * 4)
            FG_SM_LAUNCH(4);
        else if (aligned && C4 <= kNT * 16)
            FG_SM_LAUNCH(16);
        else if (aligned && C4 <= kNT * 32)
            FG_SM_LAUNCH(32);
        else
            softmax_rows_stream<<<grid, block, 0, st>>>(x, ldx, labels, C, scale, row_loss, out,
                                                        ldo, argmax, dt, probs, ldp);
#undef FG_SM_LAUNCH
    }
    FG_LAUNCH_CHECK("softmax_rows");
    return FG_OK;
}

}  // namespace

namespace fg {
int launch_mean_loss(hipStream_t stream, const float *d_row_loss, int R, float *d_mean_loss) {
    FG_REQUIRE(d_row_loss && d_mean_loss && R >= 0, FG_ERR_INVALID_ARGUMENT,
               "launch_mean_loss: NULL buffer or negative row count");
    mean_kernel<<<1, 1024, 0, stream>>>(d_row_loss, R, d_mean_loss);
    FG_LAUNCH_CHECK("mean_kernel");
    return FG_OK;
}

int softmax_ce_dispatches(int R, int C, bool mean) {
    const bool small = small_case(R, C);
    return (mean && !small) ? 2 : 1;
}

bool softmax_ce_row16_case(int R, int C) { return tiny_case(R, C); }

int softmax_ce_ex(fg_ctx *ctx, int dtype, const void *d_logits, int ldx, const uint32_t *d_labels,
                  int R, int C, float grad_scale, float *d_row_loss, float *d_mean_loss,
                  void *d_dlogits, int ldd, uint32_t *d_argmax, void *d_probs, int ldp) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "fg_softmax_ce: ctx is NULL");
    FG_REQUIRE(dtype >= FG_DTYPE_F32 && dtype <= FG_DTYPE_BF16, FG_ERR_INVALID_ARGUMENT,
               "fg_softmax_ce: bad dtype %d", dtype);
    FG_REQUIRE(R >= 0 && C > 0 && ldx >= C, FG_ERR_SHAPE,
               "fg_softmax_ce: bad shape R=%d C=%d ldx=%d", R, C, ldx);
    FG_REQUIRE(!d_dlogits || ldd >= C, FG_ERR_SHAPE, "fg_softmax_ce: ldd=%d < C=%d", ldd, C);
    FG_REQUIRE(!d_probs || ldp >= C, FG_ERR_SHAPE, "fg_softmax_ce: ldp=%d < C=%d", ldp, C);
    FG_REQUIRE(d_logits && d_labels, FG_ERR_INVALID_ARGUMENT,
               "fg_softmax_ce: logits and labels are required");
    if (R == 0) return FG_OK;
    FG_HIP(hipSetDevice(ctx->device));
    const bool small = small_case(R, C);
    float *row_loss = d_row_loss;
    if (!row_loss && d_mean_loss && !small) {
        row_loss = (float *)fg::workspace(ctx, (uint64_t)R * sizeof(float));
        if (!row_loss) return FG_ERR_OUT_OF_MEMORY;
    }
    bool mean_done = false;
    int rc = launch_rows(ctx, dtype, d_logits, ldx, d_labels, R, C, grad_scale, row_loss,
                         d_dlogits, ldd, d_argmax, d_probs, ldp, d_mean_loss, &mean_done);
    if (rc) return rc;
    if (d_mean_loss && !mean_done) {
        mean_kernel<<<1, 1024, 0, ctx->stream>>>(row_loss, R, d_mean_loss);
        FG_LAUNCH_CHECK("mean_kernel");
    }
    return FG_OK;
}
}  // namespace fg

FG_API int fg_softmax_ce(fg_ctx *ctx, int dtype, const void *d_logits, int ldx,
                         const uint32_t *d_labels, int R, int C, float grad_scale,
                         float *d_row_loss, float *d_mean_loss, void *d_dlogits, int ldd,
                         uint32_t *d_argmax) {
    return fg::softmax_ce_ex(ctx, dtype, d_logits, ldx, d_labels, R, C, grad_scale, d_row_loss,
                             d_mean_loss, d_dlogits, ldd, d_argmax, nullptr, 0);
}

FG_API int fg_softmax_ce_f32(fg_ctx *ctx, const float *d_logits, int ldx, const uint32_t *d_labels,
                             int R, int C, float grad_scale, float *d_row_loss, float *d_mean_loss,
                             float *d_dlogits, int ldd, uint32_t *d_argmax) {
    return fg_softmax_ce(ctx, FG_DTYPE_F32, d_logits, ldx, d_labels, R, C, grad_scale, d_row_loss,
                         d_mean_loss, d_dlogits, ldd, d_argmax);
}

FG_API int fg_softmax(fg_ctx *ctx, int dtype, const void *d_x, int R, int C, void *d_y) {
    FG_REQUIRE(ctx && d_x && d_y, FG_ERR_INVALID_ARGUMENT, "fg_softmax: NULL argument");
    FG_REQUIRE(dtype >= FG_DTYPE_F32 && dtype <= FG_DTYPE_BF16, FG_ERR_INVALID_ARGUMENT,
               "fg_softmax: bad dtype %d", dtype);
    FG_REQUIRE(R >= 0 && C > 0, FG_ERR_SHAPE, "fg_softmax: bad shape R=%d C=%d", R, C);
    if (R == 0) return FG_OK;
    FG_HIP(hipSetDevice(ctx->device));
    return launch_rows(ctx, dtype, d_x, C, nullptr, R, C, 1.0f, nullptr, d_y, C, nullptr);
}

FG_API int fg_softmax_f32(fg_ctx *ctx, const float *d_x, int R, int C, float *d_y) {
    return fg_softmax(ctx, FG_DTYPE_F32, d_x, R, C, d_y);
}

FG_API int fg_softmax_bwd(fg_ctx *ctx, int dtype, const void *d_y, const void *d_dy, int R, int C,
                          void *d_dx, int accumulate) {
    FG_REQUIRE(ctx && d_y && d_dy && d_dx, FG_ERR_INVALID_ARGUMENT,
               "fg_softmax_bwd: NULL argument");
    FG_REQUIRE(dtype >= FG_DTYPE_F32 && dtype <= FG_DTYPE_BF16, FG_ERR_INVALID_ARGUMENT,
               "fg_softmax_bwd: bad dtype %d", dtype);
    FG_REQUIRE(R >= 0 && C > 0, FG_ERR_SHAPE, "fg_softmax_bwd: bad shape R=%d C=%d", R, C);
    if (R == 0) return FG_OK;
    FG_HIP(hipSetDevice(ctx->device));
    softmax_bwd_rows<<<R, kNT, 0, ctx->stream>>>(d_y, d_dy, C, d_dx, accumulate, dtype);
    FG_LAUNCH_CHECK("softmax_bwd_rows");
    return FG_OK;
}

FG_API int fg_softmax_bwd_f32(fg_ctx *ctx, const float *d_y, const float *d_dy, int R, int C,
                              float *d_dx, int accumulate) {
    return fg_softmax_bwd(ctx, FG_DTYPE_F32, d_y, d_dy, R, C, d_dx, accumulate);
}
