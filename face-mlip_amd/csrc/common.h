// Shared definitions for the FACE hot-path kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/face_hip.h"

#define FACE_LAUNCH_CHECK()                               \
    do {                                                  \
        hipError_t e_ = hipGetLastError();                \
        if (e_ != hipSuccess) return (int)e_;             \
    } while (0)

namespace face {

constexpr int kWave = 64;

// Rank of each of the 20 symmetric monomials (1 | x y z | 6 rank-2 | 10 rank-3).
__host__ __device__ constexpr int rank_of(int x) { return x == 0 ? 0 : (x < 4 ? 1 : (x < 10 ? 2 : 3)); }

// Edge range of receiver atom i: CSR row_ptr, or the uniform padded stride M when row_ptr is null.
__device__ __forceinline__ void row_range(const int32_t* __restrict__ row_ptr, int64_t i, int M, int64_t& e0,
                                          int64_t& e1) {
    if (row_ptr) {
        e0 = row_ptr[i];
        e1 = row_ptr[i + 1];
    } else {
        e0 = i * (int64_t)M;
        e1 = e0 + M;
    }
}

// Butterfly sum over aligned groups of `width` lanes (width a power of two <= 64); every
// lane of the group ends with the group total.
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Cross-lane data movement on the VALU (DPP), no LDS round trip: the value of the lane that the
// DPP control selects within the lane's 16-lane row (all lanes of the row active).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of 16 lanes, every lane ending with its group's total: lane ^ 1 and
// lane ^ 2 (quad permutes), then the other quad of the half row (row_half_mirror, 7 - i) and the
// other half row (row_mirror, 15 - i), which after the first two steps hold the same partial sums
// that lane ^ 4 and lane ^ 8 would: the pairing and rounding of group_sum(v, 16), bit for bit,
// in four VALU instructions instead of four LDS permutes.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);                                 // quad_perm [1, 0, 3, 2]
    v += dpp_f<0x4E>(v);                                 // quad_perm [2, 3, 0, 1]
    v += dpp_f<0x141>(v);                                // row_half_mirror
    v += dpp_f<0x140>(v);                                // row_mirror
    return v;
}

// fp32 matrix-core helpers. v_mfma_f32_16x16x4f32 operand layouts (wave64): A[i][k] in lane
// i + 16k, B[k][j] in lane j + 16k, D[4q + r][j] in register r of lane j + 16q.
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f mfma_16x16x4(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4f ld4(const float* p) { return *reinterpret_cast<const v4f*>(p); }

// float4 read of an LDS image (16-byte aligned base) at a float offset that is a multiple of 4:
// one ds_read_b128. A plain pointer cast at a runtime offset leaves the alignment unknown to
// the compiler, which then splits the read into 32-bit pairs (ds_read2_b32).
__device__ __forceinline__ v4f lds4_at(const float* base, int off) {
    return reinterpret_cast<const v4f*>(__builtin_assume_aligned(base, 16))[off >> 2];
}
__device__ __forceinline__ void st4(float* p, v4f v) { *reinterpret_cast<v4f*>(p) = v; }

// Workgroup copy of n float4 items, put(v, src(v)) for v < n, U loads per thread issued before
// their U stores: a staging loop that stores each item before loading the next one waits a
// full memory latency per round.
template <int U, typename Src, typename Put>
__device__ __forceinline__ void stage4(int n, Src src, Put put) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    for (int v0 = 0; v0 < n; v0 += U * nthr) {
        v4f b[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int v = v0 + u * nthr + tid;
            if (v < n) b[u] = src(v);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int v = v0 + u * nthr + tid;
            if (v < n) put(v, b[u]);
        }
    }
}

// LDS image of a (F, K) row-major weight block read as float4 chunks of 16 rows at a time:
// row f at f * S; with S = K (K = 32, 64) the float4 chunk c of row f is stored at chunk
// (c + f) mod K/4, otherwise S = K + 4: both keep the 16 rows read by one instruction on
// distinct banks.
__device__ __forceinline__ int lin_off(int f, int c4, int S, int nch, bool rot) {
    return f * S + 4 * (rot ? ((c4 + f) & (nch - 1)) : c4);
}

// Row stride, swizzle and row chunk of that image for an LDS budget (f_chunk < F: the block is
// split over several workgroups); false if not even 16 rows fit.
static inline bool lin_layout(int F, int K, int max_lds, int& S, int& rot, int& f_chunk) {
    const int nch = K / 4;
    if ((int64_t)F * (K + 4) * 4 <= max_lds) {
        S = K + 4, rot = 0, f_chunk = F;
    } else if ((nch & (nch - 1)) == 0 && nch >= 8 && (int64_t)F * K * 4 <= max_lds) {
        S = K, rot = 1, f_chunk = F;
    } else {
        S = K + 4, rot = 0;
        const int rows = (max_lds / (4 * S)) / 16 * 16;
        if (rows < 16) return false;
        const int nchunk = (F + rows - 1) / rows;
        f_chunk = ((F / 16 + nchunk - 1) / nchunk) * 16;
    }
    return true;
}

// Attribute of the current device, cached per device and attribute slot (fallback if the
// query fails).
template <int Slot>
static inline int device_attr(hipDeviceAttribute_t a, int fallback) {
    constexpr int kMaxDev = 64;
    static int cache[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return fallback;
    int& v = cache[dev];
    if (v <= 0 && (hipDeviceGetAttribute(&v, a, dev) != hipSuccess || v <= 0)) v = fallback;
    return v;
}
static inline int device_cu_count() { return device_attr<0>(hipDeviceAttributeMultiprocessorCount, 256); }
static inline int device_max_lds() { return device_attr<1>(hipDeviceAttributeMaxSharedMemoryPerBlock, 65536); }

}  // namespace face
