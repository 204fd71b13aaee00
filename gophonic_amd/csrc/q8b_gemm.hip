// Block-32 int8 GEMM on MI355X: BASELINE configuration 2 as worded there
// (activations and weights each with one fp32 scale per 32-value block). The
// reference has no such function: its q8gemm int8 path scales per row
// (int8.go:106-211, gphq_q8gemm_*). Each 32-value block is quantized with
// WorkspaceI8's per-row rule (int8.go:106-168), and the product sums, per
// output and in block order, acc = fmaf(float(dot_b), da[r][b] * dw[c][b], acc)
// with dot_b the exact int32 block product, so results are bit-exact against
// the oracle's restatement of that sum.
//
// v_mfma_i32_32x32x32_i8 takes exactly one 32-value block per instruction, so
// every block's int32 products come out of one MFMA with a zero accumulator;
// the fp32 scale-accumulate that follows is VALU work (three instructions per
// output and block), which bounds this kernel well below the int8 MFMA rate.
#include "common.h"

using namespace gphq;

namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// One thread per (row, 32-value block): scale = max/127 and inverse = 127/max
// (both 0 unless 0 < max < inf, int8.go:106-119), codes RNE(x * inverse)
// saturated to int8 (int8.go:163-168; a NaN product gives 0).
__global__ __launch_bounds__(256) void q8b_quantize_kernel(const float *__restrict__ x, int rows, int k, long stride,
                                                           int8_t *__restrict__ q, float *__restrict__ d) {
    const int kb = k >> 5;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)rows * kb) return;
    const int r = (int)(idx / kb), b = (int)(idx - (long)r * kb);
    const float4 *src = (const float4 *)(x + r * stride + b * 32);
    float v[32];
    float mx = 0.0f;
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = src[i];
        v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        nan |= v[i] != v[i];
        mx = fmaxf(mx, fabsf(v[i]));
    }
    float s = 0.0f, inv = 0.0f;
    if (!nan && mx > 0.0f && mx != INFINITY) {
        s = __fdiv_rn(mx, 127.0f);
        inv = __fdiv_rn(127.0f, mx);
    }
    d[idx] = s;
    int32_t packed[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float p = __fmul_rn(v[4 * w + j], inv);
            float c = p != p ? 0.0f : rintf(p);
            c = fminf(127.0f, fmaxf(-128.0f, c));
            word |= (uint32_t)(uint8_t)(int8_t)(int)c << (8 * j);
        }
        packed[w] = (int32_t)word;
    }
    int32_t *dst = (int32_t *)(q + (long)r * k + b * 32);
    *(i32x4 *)dst = i32x4{packed[0], packed[1], packed[2], packed[3]};
    *(i32x4 *)(dst + 4) = i32x4{packed[4], packed[5], packed[6], packed[7]};
}

struct Q8bArgs {
    const int8_t *qa;
    const float *da;
    const int8_t *qw;
    const float *dw;
    float *y;
    int m, k, n, gridM, gridN;
};

// BM x BN output tiles, WGM x WGN wavefronts of (BM/WGM) x (BN/WGN) as 32x32
// MFMA tiles. Per 128-byte K step (four blocks) both code tiles pass through
// LDS in 128-byte rows with XOR-swizzled 16-byte chunks (big_swz), the step's
// block scales as [block][row] floats; double buffered, the next step's global
// loads one step ahead in registers. Rows past m or n load row m-1 / n-1 and
// are not stored; blocks past k are skipped.
template <int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void q8b_gemm_kernel(const Q8bArgs a) {
    constexpr int NT = 64 * WGM * WGN;
    constexpr int TI = BM / WGM / 32, TJ = BN / WGN / 32;
    constexpr int AL = BM * 8 / NT, BL = BN * 8 / NT;  // 16-byte code units per thread and step
    static_assert(AL >= 1 && BL >= 1 && BM + BN <= NT, "loader split");
    __shared__ i32x4 As[2][BM * 8];
    __shared__ i32x4 Bs[2][BN * 8];
    __shared__ float Sa[2][4][BM];
    __shared__ float Sb[2][4][BN];
    int bm, bn;
    tile_order(blockIdx.x, a.gridM, a.gridN, bm, bn);
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int wm = wv / WGN, wn = wv % WGN;
    const int m0 = bm * BM, n0 = bn * BN;
    const int kb = a.k >> 5, steps = (kb + 3) >> 2;

    // Loader: unit u = i*NT + t is row u/8, 16-byte chunk u%8 of the step's
    // 128 bytes; chunks past k load zeros. Threads t < BM load A's scale row
    // t, threads NT-BN .. NT-1 B's scale row t-(NT-BN) (four floats each).
    i32x4 ar[AL], br[BL];
    float4 sr;
    auto gload = [&](int st) {
        const int kbyte = st * 128;
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int u = i * NT + t, row = u >> 3, ch = u & 7;
            const int gr = min(m0 + row, a.m - 1);
            ar[i] = kbyte + ch * 16 < a.k ? *(const i32x4 *)(a.qa + (long)gr * a.k + kbyte + ch * 16) : i32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            const int u = i * NT + t, row = u >> 3, ch = u & 7;
            const int gr = min(n0 + row, a.n - 1);
            br[i] = kbyte + ch * 16 < a.k ? *(const i32x4 *)(a.qw + (long)gr * a.k + kbyte + ch * 16) : i32x4{0, 0, 0, 0};
        }
        const int b0 = st * 4;
        sr = float4{0.f, 0.f, 0.f, 0.f};
        const float *srow = nullptr;
        if (t < BM)
            srow = a.da + (long)min(m0 + t, a.m - 1) * kb;
        else if (t >= NT - BN)
            srow = a.dw + (long)min(n0 + t - (NT - BN), a.n - 1) * kb;
        if (srow) {
            sr.x = srow[b0];
            if (b0 + 1 < kb) sr.y = srow[b0 + 1];
            if (b0 + 2 < kb) sr.z = srow[b0 + 2];
            if (b0 + 3 < kb) sr.w = srow[b0 + 3];
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int u = i * NT + t, row = u >> 3;
            As[buf][row * 8 + big_swz(row, u & 7)] = ar[i];
        }
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            const int u = i * NT + t, row = u >> 3;
            Bs[buf][row * 8 + big_swz(row, u & 7)] = br[i];
        }
        if (t < BM) {
            Sa[buf][0][t] = sr.x, Sa[buf][1][t] = sr.y, Sa[buf][2][t] = sr.z, Sa[buf][3][t] = sr.w;
        } else if (t >= NT - BN) {
            const int r = t - (NT - BN);
            Sb[buf][0][r] = sr.x, Sb[buf][1][r] = sr.y, Sb[buf][2][r] = sr.z, Sb[buf][3][r] = sr.w;
        }
    };

    f32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x16{};
    gload(0);
    lstore(0);
    if (steps > 1) gload(1);
    __syncthreads();
    const int fr = lane & 31, fh = lane >> 5;
    for (int st = 0; st < steps; ++st) {
        const int cur = st & 1;
        const int nb = min(4, kb - st * 4);
        auto block = [&](int b) {
            const int c = 2 * b + fh;
            i32x4 fa[TI], fb[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const int r = wm * (32 * TI) + 32 * i + fr;
                fa[i] = As[cur][r * 8 + big_swz(r, c)];
            }
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int r = wn * (32 * TJ) + 32 * j + fr;
                fb[j] = Bs[cur][r * 8 + big_swz(r, c)];
            }
            // Scales: this lane's 16 result rows of tile i are 4 runs of 4
            // consecutive rows; its column's weight scale is one float.
            float4 sa[TI][4];
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    sa[i][q] = *(const float4 *)&Sa[cur][b][wm * (32 * TI) + 32 * i + 8 * q + 4 * fh];
            float sb[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j) sb[j] = Sb[cur][b][wn * (32 * TJ) + 32 * j + fr];
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const i32x16 dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], i32x16{}, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float s4[4] = {sa[i][q].x, sa[i][q].y, sa[i][q].z, sa[i][q].w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float s = __fmul_rn(s4[e], sb[j]);
                            acc[i][j][4 * q + e] = __builtin_fmaf((float)dot[4 * q + e], s, acc[i][j][4 * q + e]);
                        }
                    }
                }
        };
        // Unrolled over a full step for one tile per wavefront; with more the
        // registers of four blocks in flight cost more than the overlap gains.
        if (TI * TJ == 1 && nb == 4) {
#pragma unroll
            for (int b = 0; b < 4; ++b) block(b);
        } else {
            for (int b = 0; b < nb; ++b) block(b);
        }
        if (st + 1 < steps) {
            lstore(cur ^ 1);
            if (st + 2 < steps) gload(st + 2);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int col = n0 + wn * (32 * TJ) + 32 * j + fr;
            if (col >= a.n) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * (32 * TI) + 32 * i + 8 * (e >> 2) + 4 * fh + (e & 3);
                if (row < a.m) a.y[(long)row * a.n + col] = acc[i][j][e];
            }
        }
}

// M <= 2 (K a multiple of 1024): one wavefront per group of kRowsRW weight
// rows, so the grid is N / 4 blocks wide instead of N / 128. Lane l takes
// 16-byte chunk l of each 1 KiB K step of its rows and of every activation
// row; v_dot4_i32_i8 gives exact int32 partial dots, lanes l and l ^ 1 add
// their halves into the 32-value block's dot (exact), which is staged in LDS
// with both scale vectors. Lane (r, i) then runs output (i, row r)'s chain
// acc = fmaf(float(dot_b), da[i][b] * dw[r][b], acc) in block order: the
// operations of the tiled kernel and of the oracle, so the result is the same
// bit for bit.
constexpr int kRowsRW = 4;
// Each activation row adds a pass over the lane's K chunks and a chain per
// output: measured at K = 4096, N = 12288, M = 1 takes 23 us (the tiled
// kernel 47 us) and M = 16 192 us, so the kernel stops at two rows.
constexpr int kRowsMaxM = 2;
__global__ __launch_bounds__(64) void q8b_rows_kernel(const Q8bArgs a) {
    extern __shared__ float sm[];
    const int KB = a.k >> 5, m = a.m, lane = threadIdx.x;
    float *dots = sm;                     // [kRowsRW][m][KB]
    float *sw = dots + kRowsRW * m * KB;  // [kRowsRW][KB] weight block scales
    float *sa = sw + kRowsRW * KB;        // [m][KB] activation block scales
    const int n0 = blockIdx.x * kRowsRW;
    for (int i = lane; i < kRowsRW * KB; i += 64) {
        const int r = i / KB, b = i - r * KB;
        sw[i] = a.dw[(size_t)min(n0 + r, a.n - 1) * KB + b];
    }
    for (int i = lane; i < m * KB; i += 64) sa[i] = a.da[i];
    const int steps = a.k >> 10;
    for (int s = 0; s < steps; ++s) {
        const size_t kb = (size_t)s * 1024 + (size_t)lane * 16;
        i32x4 w[kRowsRW];
#pragma unroll
        for (int r = 0; r < kRowsRW; ++r) w[r] = *(const i32x4 *)(a.qw + (size_t)min(n0 + r, a.n - 1) * a.k + kb);
        for (int i = 0; i < m; ++i) {
            const i32x4 x = *(const i32x4 *)(a.qa + (size_t)i * a.k + kb);
#pragma unroll
            for (int r = 0; r < kRowsRW; ++r) {
                int d = __builtin_amdgcn_sdot4(x.x, w[r].x, 0, false);
                d = __builtin_amdgcn_sdot4(x.y, w[r].y, d, false);
                d = __builtin_amdgcn_sdot4(x.z, w[r].z, d, false);
                d = __builtin_amdgcn_sdot4(x.w, w[r].w, d, false);
                d += __shfl_xor(d, 1);
                if (!(lane & 1)) dots[(r * m + i) * KB + s * 32 + (lane >> 1)] = (float)d;
            }
        }
    }
    __syncthreads();
    if (lane < kRowsRW * m) {
        const int r = lane / m, i = lane - r * m;
        const float *dr = dots + (r * m + i) * KB, *wr = sw + r * KB, *ar = sa + i * KB;
        float acc = 0.0f;
        for (int b = 0; b < KB; ++b) acc = fmaf(dr[b], ar[b] * wr[b], acc);
        if (n0 + r < a.n) a.y[(size_t)i * a.n + n0 + r] = acc;
    }
}

size_t rows_lds_bytes(int m, int k) { return (size_t)(kRowsRW * m + kRowsRW + m) * (k / 32) * 4; }

template <int BM, int BN, int WGM, int WGN>
int launch_q8b(Q8bArgs a, hipStream_t st) {
    a.gridM = (a.m + BM - 1) / BM;
    a.gridN = (a.n + BN - 1) / BN;
    hipLaunchKernelGGL((q8b_gemm_kernel<BM, BN, WGM, WGN>), dim3((unsigned)(a.gridM * a.gridN)),
                       dim3(64 * WGM * WGN), 0, st, a);
    return launch_status();
}

}  // namespace

extern "C" {

int gphq_q8b_quantize(const float *x_dev, int64_t rows, int64_t k, int64_t x_stride, int8_t *q_dev, float *d_dev,
                      void *stream) {
    if (rows < 0 || k < 0 || k % 32 || x_stride < k || x_stride % 4 || rows > INT32_MAX || k > INT32_MAX)
        return GPHQ_ERR_DIMENSIONS;
    if (rows == 0 || k == 0) return GPHQ_OK;
    if (!x_dev || !q_dev || !d_dev) return GPHQ_ERR_DIMENSIONS;
    const long items = (long)rows * (k / 32);
    hipLaunchKernelGGL(q8b_quantize_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       x_dev, (int)rows, (int)k, (long)x_stride, q_dev, d_dev);
    return launch_status();
}

int gphq_q8b_gemm(const int8_t *qa_dev, const float *da_dev, const int8_t *qw_dev, const float *dw_dev, float *y_dev,
                  int64_t m, int64_t k, int64_t n, void *stream) {
    if (m < 0 || k < 0 || n < 0 || k % 32 || m > INT32_MAX || k > INT32_MAX || n > INT32_MAX)
        return GPHQ_ERR_DIMENSIONS;
    if (m == 0 || n == 0) return GPHQ_OK;
    if (!qa_dev || !da_dev || !qw_dev || !dw_dev || !y_dev) return GPHQ_ERR_DIMENSIONS;
    if (k == 0) return fill_f32(y_dev, (size_t)m * n, 0.0f, (hipStream_t)stream);
    Q8bArgs a{qa_dev, da_dev, qw_dev, dw_dev, y_dev, (int)m, (int)k, (int)n, 0, 0};
    hipStream_t st = (hipStream_t)stream;
    // 128 x 128 tiles from M = 256; below, 32-row tiles keep the grid wide;
    // up to 2 rows, the dot-product kernel.
    if (m >= 256) return launch_q8b<128, 128, 2, 2>(a, st);
    if (m <= kRowsMaxM && k % 1024 == 0 && rows_lds_bytes((int)m, (int)k) <= 65536) {
        hipLaunchKernelGGL(q8b_rows_kernel, dim3((unsigned)((n + kRowsRW - 1) / kRowsRW)), dim3(64),
                           rows_lds_bytes((int)m, (int)k), st, a);
        return launch_status();
    }
    return launch_q8b<32, 128, 1, 4>(a, st);
}

}  // extern "C"
