// Shared helpers for libgphq: error codes, launch checks, wavefront reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>
#include <vector>

#include "../../include/gphq.h"

namespace gphq {

// Records the most recent HIP failure so gphq_last_hip_error() can report it.
void set_hip_error(hipError_t e);

// Converts a HIP status into a gphq status, remembering the HIP code.
inline int hip_status(hipError_t e) {
    if (e == hipSuccess) return GPHQ_OK;
    set_hip_error(e);
    return GPHQ_ERR_HIP;
}

// Checks the launch that was just enqueued.
inline int launch_status() { return hip_status(hipGetLastError()); }

// A K-split multi-vector GEMV whose residual add is left to the next
// activation preparation: its parts [parts][V][N], its vectors' scales and,
// for Q8, its row scales. parts == 0: nothing pending.
struct VecFold {
    const float *part = nullptr;
    const float *inv = nullptr;
    const float *rowScale = nullptr;
    int parts = 0;
};

// Compute units of the current device (cached per device).
inline int device_cus() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// A grid of rows256 x cols256 tiles of 256 x 256 outputs that is not a whole
// number of rounds of the chip (one tile per CU): the number of 256-wide
// column tiles, from the left, whose tiles fill whole rounds (0 when the
// grid is whole rounds already or smaller than one).
inline long whole_round_cols256(long rows256, long cols256) {
    const long cus = device_cus(), big = rows256 * cols256;
    if (big % cus == 0 || big < cus) return 0;
    const long full = (big / cus) * cus / rows256;
    return full < cols256 ? full : 0;
}

// n floats of dst set to v by a fill kernel (util.hip); never hipMemsetAsync,
// so the fill may be captured in a HIP graph.
int fill_f32(float *dst, size_t n, float v, hipStream_t stream);

#define GPHQ_TRY(expr)                      \
    do {                                    \
        int _st = (expr);                   \
        if (_st != GPHQ_OK) return _st;     \
    } while (0)

// ---- device helpers --------------------------------------------------------

// Butterfly sum inside each row of 16 lanes, using DPP lane permutes, so every
// lane of a row ends with that row's total. quad_perm [1,0,3,2] and [2,3,0,1]
// pair lanes at distance 1 and 2; row_half_mirror pairs the two quads of an
// 8-lane half; row_mirror pairs the two halves of a row.
__device__ __forceinline__ float row16_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
    return v;
}

// Sum over the 64 lanes of a wavefront; the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (a + b) + (c + d);
}

// One round of lds_fwht: the R = 2^r stages h = 2^s .. 2^(s+r-1) at once.
// Each item owns the R values whose index differs only in bits s..s+r-1
// (base = idx with r zero bits inserted at bit s), runs the r stages on them
// in registers, stage by stage in the network's order, and stores them back.
// With PAD, value i lives at LDS word rot_pad(i): 16 words of padding per 256
// values, so the four 16-item groups of a wavefront at stride 16 fall on
// different banks, and the four 16-byte quads of each 16-value chunk rotated
// by (i / 64) % 4, so 16 lanes storing or loading consecutive chunks 16 bytes
// at a time cover all 64 banks once. Within 64 consecutive values the map is
// a permutation, so rounds with a stride of 64 or more stay conflict-free.
__device__ __forceinline__ int rot_pad(int i) {
    return (i & ~15) + ((((i >> 2) + (i >> 6)) & 3) << 2) + (i & 3) + ((i >> 8) << 4);
}

// NT: the block's thread count when the caller knows it (blockDim.x is read
// from the dispatch packet, a memory round trip, at every use); 0 for any.
template <int R, bool PAD = false, int NT = 0>
__device__ __forceinline__ void fwht_round(float *v, int n, int s) {
    constexpr int r = R == 16 ? 4 : R == 8 ? 3 : R == 4 ? 2 : 1;
    const int h = 1 << s;
    const int nt = NT ? NT : (int)blockDim.x;
    for (int idx = threadIdx.x; idx < (n >> r); idx += nt) {
        const int base = ((idx >> s) << (s + r)) | (idx & (h - 1));
        float a[R];
#pragma unroll
        for (int j = 0; j < R; ++j) a[j] = v[PAD ? rot_pad(base + j * h) : base + j * h];
#pragma unroll
        for (int m = 1; m < R; m <<= 1)
#pragma unroll
            for (int j = 0; j < R; ++j)
                if (!(j & m)) {
                    const float x = a[j], y = a[j + m];
                    a[j] = x + y;
                    a[j + m] = x - y;
                }
#pragma unroll
        for (int j = 0; j < R; ++j) v[PAD ? rot_pad(base + j * h) : base + j * h] = a[j];
    }
    __syncthreads();
}

// In-place unnormalized Walsh-Hadamard transform of each `block` run of
// v[0..n) in LDS (block a power of two dividing n), stages h = 1, 2, 4, ...:
// the butterfly network of qwen3lm/hadamard.go:62-78. Every value goes
// through the same additions in the same order as in the sequential network,
// so the fp32 result equals it bit for bit; three stages share one pass over
// LDS. All threads of the block take part; the caller has made v visible
// (barrier) before the call, and the call ends with a barrier.
__device__ inline void lds_fwht(float *v, int n, int block) {
    const int lb = __builtin_ctz((unsigned)block);
    int s = 0;
    for (; s + 3 <= lb; s += 3) fwht_round<8>(v, n, s);
    if (lb - s == 2) fwht_round<4>(v, n, s);
    if (lb - s == 1) fwht_round<2>(v, n, s);
}

// A row held in registers by a one-block-per-row kernel of 256 threads
// (thread t owns chunks of 16 values at 16 * (t + 256 c), c < CPT; chunks
// past K are left as they are) is rotated in place: x * signs (the scale
// folded into signs), then lds_fwht over the row in blocks of `block`, in
// rot_lds_bytes(K) of dynamic LDS (a segment padded by rot_pad).
//
// Chunk c of every thread is segment c of the row, values 4096c .. 4096c +
// 4095, and a block (a power of two up to 4096 dividing K) never straddles
// two segments, so the segments are rotated one after another through the
// same LDS: 16.6 KB however long the row (a 12288-value row took 49.9 KB,
// which left room for three rows per CU). The network's first stages (h = 1
// .. 8, up to the block) pair values of one thread's 16-value chunk, so they
// run in registers before the segment goes to LDS; the rest run as radix-16
// rounds (then 8, 4, 2) from stage h = 16, whose 16 consecutive items read
// consecutive words. Same butterflies in the same stage order as lds_fwht, so
// the same bits.
inline size_t rot_lds_bytes(int K) {
    const int n = K < 4096 ? K : 4096;
    return (size_t)(n + (n >> 8) * 16 + 16) * sizeof(float);
}

// The signs of a thread's chunk at k (clamped into the row), for
// rotate_row_lds: the caller loads segment 0's before the row itself, so the
// first segment waits only for its own loads.
__device__ __forceinline__ void rot_signs(float4 (&sg)[4], const float *__restrict__ signs, int k, int K) {
    const int kk = k < K - 16 ? k : K - 16;
#pragma unroll
    for (int q = 0; q < 4; ++q) sg[q] = *(const float4 *)(signs + kk + 4 * q);
}

// The two radix-16 rounds of a 4096-value block (stages h = 16 .. 2048) over
// 256 threads, on the rot_pad layout, with each thread's addresses in closed
// form: in the round from h = 16, thread t owns values 256 (t >> 4) + (t & 15)
// + 16 j, which sit at words A + 64 (j >> 2) + 16 (j & 3) + 4 ((q + (j >> 2))
// & 3) (A = 272 (t >> 4) + (t & 3), q = (t >> 2) & 3); in the round from
// h = 256 it owns t + 256 j, at rot_pad(t) + 272 j. The same words, items and
// butterflies as two fwht_round<16, true, 256> calls (s = 4, 8), so the same
// bits; the generic rounds recompute rot_pad for every access.
__device__ __forceinline__ void fwht4096_rounds_pad(float *v) {
    const int t = (int)threadIdx.x;
    float a[16];
    auto butterflies = [&]() {
#pragma unroll
        for (int m = 1; m < 16; m <<= 1)
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (!(j & m)) {
                    const float x = a[j], y = a[j + m];
                    a[j] = x + y;
                    a[j + m] = x - y;
                }
    };
    {
        const int A = 272 * (t >> 4) + (t & 3), q = (t >> 2) & 3;
        int base[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) base[m] = A + 64 * m + (((q + m) & 3) << 2);
#pragma unroll
        for (int j = 0; j < 16; ++j) a[j] = v[base[j >> 2] + 16 * (j & 3)];
        butterflies();
#pragma unroll
        for (int j = 0; j < 16; ++j) v[base[j >> 2] + 16 * (j & 3)] = a[j];
        __syncthreads();
    }
    {
        const int b = rot_pad(t);
#pragma unroll
        for (int j = 0; j < 16; ++j) a[j] = v[b + 272 * j];
        butterflies();
#pragma unroll
        for (int j = 0; j < 16; ++j) v[b + 272 * j] = a[j];
        __syncthreads();
    }
}

template <int CPT>
__device__ __forceinline__ void rotate_row_lds(float4 (&v)[CPT][4], float4 (&sg)[4], int K,
                                               const float *__restrict__ signs, int block) {
    extern __shared__ float rot_lds[];
    const int lb = __builtin_ctz((unsigned)block);
    const int kl = 16 * (int)threadIdx.x;  // the thread's chunk within a segment
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int seg = 4096 * c;
        if (c > 0 && seg >= K) break;  // (K >= 16: segment 0 always exists)
        const int n = K - seg < 4096 ? K - seg : 4096;
        const int k = seg + kl;
        if (c > 0) __syncthreads();  // the previous segment has been read back
        float a[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            a[4 * q] = v[c][q].x * sg[q].x;
            a[4 * q + 1] = v[c][q].y * sg[q].y;
            a[4 * q + 2] = v[c][q].z * sg[q].z;
            a[4 * q + 3] = v[c][q].w * sg[q].w;
        }
        if (c + 1 < CPT && seg + 4096 < K) rot_signs(sg, signs, k + 4096, K);  // the next segment's
        if (k < K) {
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) {
                if (m >= block) break;
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (!(j & m)) {
                        const float x = a[j], y = a[j + m];
                        a[j] = x + y;
                        a[j + m] = x - y;
                    }
            }
            // Each quad of 4 values stays contiguous under rot_pad.
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *(float4 *)(rot_lds + rot_pad(kl + 4 * q)) = float4{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
        }
        __syncthreads();
        int s = 4;
        if (n == 4096 && lb == 12) {  // whole 4096-value blocks: both rounds with closed-form addresses
            fwht4096_rounds_pad(rot_lds);
            s = 12;
        }
        for (; s + 4 <= lb; s += 4) fwht_round<16, true, 256>(rot_lds, n, s);
        if (lb - s == 3) fwht_round<8, true, 256>(rot_lds, n, s);
        if (lb - s == 2) fwht_round<4, true, 256>(rot_lds, n, s);
        if (lb - s == 1) fwht_round<2, true, 256>(rot_lds, n, s);
        if (k < K) {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[c][q] = *(const float4 *)(rot_lds + rot_pad(kl + 4 * q));
        }
    }
}

// Chunk c of a 256-thread row kernel: 16 values at k = 16 * (t + 256 c)
// (K % 16 == 0). The load is issued on every path (the address clamped into
// the row), so the compiler's waits count only the loads issued before the
// ones a use needs; chunks past K hold a copy of the last chunk until
// zero_past_end, which the kernel calls where it first needs the values.
template <int CPT>
__device__ __forceinline__ void load_row_chunks(float4 (&v)[CPT][4], const float *__restrict__ xr, int K) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int k = 16 * ((int)threadIdx.x + 256 * c);
        const int kk = k < K - 16 ? k : K - 16;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = *(const float4 *)(xr + kk + 4 * q);
    }
}

template <int CPT>
__device__ __forceinline__ void zero_past_end(float4 (&v)[CPT][4], int K) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        if (16 * ((int)threadIdx.x + 256 * c) < K) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = float4{0.f, 0.f, 0.f, 0.f};
    }
}

// qwen3lm/hadamard.go:24-47 newRotation(k): fills k signs (+-1) and returns
// the block (the largest power of two up to 4096 dividing k); the scale is
// 1/sqrt(block) rounded to float32.
int rotation_signs_pm1(int64_t k, std::vector<float> &signs);
inline float rotation_scale(int64_t block) { return (float)(1.0 / __builtin_sqrt((double)block)); }

// IEEE half bits -> float (exact), for FP16 scales stored as raw uint16.
__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// ---- int8 activation quantization (WorkspaceI8) --------------------------------

// quantize (int8.go:163-168): round half to even, saturate; a NaN (x * 0 for a
// non-finite row) converts to 0, as Go's float->int8 conversion does on amd64
// and arm64.
__device__ __forceinline__ int8_t quantize_i8(float v) {
    if (v != v) return 0;
    const float r = rintf(v);
    return (int8_t)fminf(fmaxf(r, -128.0f), 127.0f);
}

// SetRowScale (int8.go:106-112): max/127 and 127/max for finite positive max,
// else 0 and 0. fp32 division is correctly rounded (hipcc default).
__device__ __forceinline__ void i8_row_scale(float m, float &scale, float &inv) {
    if (m > 0.0f && !isinf(m) && m == m) {
        scale = m / 127.0f;
        inv = 127.0f / m;
    } else {
        scale = 0.0f;
        inv = 0.0f;
    }
}

// ---- GEMM tiling helpers ------------------------------------------------------

// Block b's output tile (bm, bn). Workgroups are dispatched to the 8 XCDs
// round robin, so XCD x = b % 8 runs blocks x, x + 8, ...; those take one
// contiguous range of the tile order, and the order walks groups of 8 M
// blocks for each N block, so the blocks an XCD runs at once share their A
// rows and B columns in that XCD's L2.
__device__ __forceinline__ void tile_order(int b, int gridM, int gridN, int &bm, int &bn) {
    constexpr int GM = 8;
    const int G = gridM * gridN;
    const int L = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
    const int span = GM * gridN;
    const int grp = L / span, first = grp * GM;
    const int gm = min(gridM - first, GM);
    const int r = L - grp * span;
    bm = first + r % gm;
    bn = r / gm;
}

// vmcnt(N) and lgkmcnt(0), expcnt untouched (gfx9 s_waitcnt encoding: vmcnt
// in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// s_barrier between compiler-only memory barriers: the builtin alone is not a
// memory operation to LLVM, so LDS reads of a ring slot could otherwise be
// moved across it. The empty asm emits no instruction and no wait count, so
// loads issued before it stay in flight.
__device__ __forceinline__ void ring_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One 16-byte-per-lane direct-to-LDS load (global_load_lds_dwordx4): lane l
// writes its 16 bytes from `src` to lds + 16 l. `lds` is the same for every
// lane. Counts in vmcnt like any vector load.
__device__ __forceinline__ void lds_dma16(const void *src, void *lds) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                     (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}

// 16-byte chunk index within a 128-byte LDS row of a GEMM operand tile,
// swizzled by the row: fragment reads of 8 or 16 consecutive rows at one
// chunk hit distinct banks.
__device__ __forceinline__ int big_swz(int row, int chunk) { return chunk ^ ((row ^ (row >> 3)) & 7); }

}  // namespace gphq
