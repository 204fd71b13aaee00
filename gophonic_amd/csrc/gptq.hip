// GPTQ producer on MI355X: the core of cmd/qwen3-gptq, qwen3lm quantizeGroup
// (gptq.go:604-666) with gptqInverseFactor (gptq_linalg.go:68-223) and
// gptqRound (gptq.go:671-796), for one group of projections sharing their
// calibration inputs.
//
//   factor: H = X^T X over the calibration rows; dead channels (H[i][i] == 0)
//     get H[i][i] = 1; H += 0.01 * mean(diag) * I; U = J chol(J H J)^-1 J, the
//     upper factor with H^-1 = U^T U. The Cholesky factorization runs in
//     64-column panels (diagonal block in one workgroup with float64 sums,
//     panel rows by forward substitution, the trailing update as an fp32
//     product); L^-1 runs in 64-row blocks (an fp32 product with the rows
//     already inverted, then the block's rows by substitution).
//   round: per 128-column block, one wavefront per weight row quantizes the
//     block's columns in order (code = clamp(rne(w / s)), error
//     e = (w - q s) / U[c][c], the block's later columns w[j] -= e U[c][j]),
//     choosing each 4-bit group's scale (q4GroupScale) from the current values
//     at the group's first column; then the columns after the block take the
//     lazy update W -= E U (an fp32 product).
// All products are fp32 with fp32 storage, as the reference's; the small
// substitutions sum in float64, as the reference's do.
#include <math.h>

#include <algorithm>
#include <vector>

#include "common.h"

using namespace gphq;

namespace {

constexpr int kPanel = 64;      // Cholesky / inverse panel width
constexpr int kRoundBlock = 128;  // gptqBlock (gptq.go:37)
constexpr int kRowsPerBlock = 8;  // weight rows (wavefronts) per rounding workgroup

// ---- fp32 product: C = [C +] alpha * op(A) op(B) ---------------------------
// A(i,p) = a[i*lda + p] (TA 0) or a[p*lda + i] (TA 1); B(p,j) = b[p*ldb + j]
// (TB 0) or b[j*ldb + p] (TB 1). 64 x 64 tiles, 256 threads with 4 x 4
// outputs each, 16-deep K chunks through LDS. lower: only j <= i is written.
// With accumulate the full sum is formed first and added once.
template <int TA, int TB>
__global__ __launch_bounds__(256) void sgemm_kernel(int M, int N, int K, float alpha, const float *__restrict__ a,
                                                    long lda, const float *__restrict__ b, long ldb, float *c,
                                                    long ldc, int accumulate, int lower) {
    __shared__ float As[16][68], Bs[16][68];
    const int bi = blockIdx.y * 64, bj = blockIdx.x * 64;
    if (lower && bj > bi + 63) return;
    const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
    float acc[4][4] = {};
    for (int p0 = 0; p0 < K; p0 += 16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = t + 256 * e;
            int i, p, j, q;
            if (TA == 0) {
                i = idx >> 4;
                p = idx & 15;
            } else {
                p = idx >> 6;
                i = idx & 63;
            }
            float va = 0.0f;
            if (bi + i < M && p0 + p < K)
                va = TA == 0 ? a[(size_t)(bi + i) * lda + p0 + p] : a[(size_t)(p0 + p) * lda + bi + i];
            As[p][i] = va;
            if (TB == 0) {
                q = idx >> 6;
                j = idx & 63;
            } else {
                j = idx >> 4;
                q = idx & 15;
            }
            float vb = 0.0f;
            if (bj + j < N && p0 + q < K)
                vb = TB == 0 ? b[(size_t)(p0 + q) * ldb + bj + j] : b[(size_t)(bj + j) * ldb + p0 + q];
            Bs[q][j] = vb;
        }
        __syncthreads();
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            float x[4], y[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                x[r] = As[p][ty * 4 + r];
                y[r] = Bs[p][tx * 4 + r];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int s = 0; s < 4; ++s) acc[r][s] = fmaf(x[r], y[s], acc[r][s]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int i = bi + ty * 4 + r, j = bj + tx * 4 + s;
            if (i >= M || j >= N || (lower && j > i)) continue;
            const float v = alpha * acc[r][s];
            float *p = c + (size_t)i * ldc + j;
            *p = accumulate ? *p + v : v;
        }
}

template <int TA, int TB>
int sgemm(int M, int N, int K, float alpha, const float *a, long lda, const float *b, long ldb, float *c, long ldc,
          bool accumulate, bool lower, hipStream_t st) {
    if (M <= 0 || N <= 0) return GPHQ_OK;
    hipLaunchKernelGGL((sgemm_kernel<TA, TB>), dim3((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64)),
                       dim3(256), 0, st, M, N, K, alpha, a, lda, b, ldb, c, ldc, accumulate ? 1 : 0, lower ? 1 : 0);
    return launch_status();
}

// Dead channels and damping (gptq.go:623-637): one block; the diagonal's mean
// in float64.
__global__ __launch_bounds__(1024) void gptq_damp_kernel(float *h, int n, uint8_t *dead) {
    __shared__ double part[16];
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += (double)h[(size_t)i * n + i];
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    double mean = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) mean += part[w];
    mean /= (double)n;
    const float add = (float)(0.01 * mean);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float d = h[(size_t)i * n + i];
        const bool isDead = d == 0.0f;
        dead[i] = isDead ? 1 : 0;
        if (isDead) d = 1.0f;
        h[(size_t)i * n + i] = d + add;
    }
}

// dst = J src J (both n x n): dst[i][j] = src[n-1-i][n-1-j].
__global__ void reverse_kernel(const float *__restrict__ src, float *__restrict__ dst, int n) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)n * n) return;
    const int i = (int)(idx / n), j = (int)(idx - (size_t)i * n);
    dst[idx] = src[(size_t)(n - 1 - i) * n + (n - 1 - j)];
}

// Factors the b x b diagonal block at j0 (already updated by earlier panels)
// in place, choleskyLower's inner loop (gptq_linalg.go:73-93): float64 sums,
// float64 pivot roots, float32 storage. Sets *bad on a non-positive pivot.
__global__ __launch_bounds__(64) void chol_diag_kernel(float *a, int n, int j0, int b, int *bad) {
    __shared__ float L[kPanel][kPanel + 1];
    __shared__ double piv;
    const int t = threadIdx.x;
    if (t < b)
        for (int p = 0; p <= t; ++p) L[t][p] = a[(size_t)(j0 + t) * n + j0 + p];
    __syncthreads();
    for (int j = 0; j < b; ++j) {
        if (t == j) {
            double d = 0.0;
            for (int p = 0; p < j; ++p) d += (double)L[j][p] * (double)L[j][p];
            d = (double)L[j][j] - d;
            if (!(d > 0.0)) {
                *bad = 1;
                d = 1.0;
            }
            piv = sqrt(d);
            L[j][j] = (float)piv;
        }
        __syncthreads();
        if (t > j && t < b) {
            double s = 0.0;
            for (int p = 0; p < j; ++p) s += (double)L[t][p] * (double)L[j][p];
            L[t][j] = (float)(((double)L[t][j] - s) / piv);
        }
        __syncthreads();
    }
    if (t < b)
        for (int p = 0; p <= t; ++p) a[(size_t)(j0 + t) * n + j0 + p] = L[t][p];
}

// Panel rows below the diagonal block: L21 = A21 L11^-T row by row
// (gptq_linalg.go:97-110), one thread per row, float64 sums.
__global__ __launch_bounds__(256) void chol_panel_kernel(float *a, int n, int j0, int b) {
    __shared__ float L[kPanel][kPanel + 1];
    for (int e = threadIdx.x; e < b * b; e += blockDim.x) {
        const int r = e / b, p = e - r * b;
        L[r][p] = p <= r ? a[(size_t)(j0 + r) * n + j0 + p] : 0.0f;
    }
    __syncthreads();
    const int i = j0 + b + (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= n) return;
    float *row = a + (size_t)i * n + j0;
    float v[kPanel];
#pragma unroll
    for (int j = 0; j < kPanel; ++j) v[j] = j < b ? row[j] : 0.0f;
#pragma unroll
    for (int j = 0; j < kPanel; ++j) {
        if (j >= b) break;
        double s = (double)v[j];
#pragma unroll
        for (int p = 0; p < kPanel; ++p)
            if (p < j) s -= (double)v[p] * (double)L[j][p];
        v[j] = (float)(s / (double)L[j][j]);
    }
#pragma unroll
    for (int j = 0; j < kPanel; ++j)
        if (j < b) row[j] = v[j];
}

// Rows i0 .. i0+b-1 of X = L^-1 (lower), every column c <= i: X[i][c] =
// (delta(i,c) - sum_{p<i} L[i][p] X[p][c]) / L[i][i], the part p < i0 given
// as T[r][c] (an fp32 product), the rest summed here in float64 over the
// block's earlier rows (invertLowerTransposed, gptq_linalg.go:141-176). One
// thread per column; X's columns of the block's rows kept in LDS.
__global__ __launch_bounds__(256) void inv_rows_kernel(const float *__restrict__ l, float *__restrict__ x,
                                                       const float *__restrict__ tt, int n, int i0, int b) {
    __shared__ float Lb[kPanel][kPanel + 1];
    __shared__ float xs[kPanel][256];
    for (int e = threadIdx.x; e < b * b; e += blockDim.x) {
        const int r = e / b, p = e - r * b;
        Lb[r][p] = p <= r ? l[(size_t)(i0 + r) * n + i0 + p] : 0.0f;
    }
    __syncthreads();
    const int c = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (c >= i0 + b) return;
    for (int r = 0; r < b; ++r) {
        const int i = i0 + r;
        float v = 0.0f;
        if (c <= i) {
            double s = c < i0 ? (double)tt[(size_t)r * i0 + c] : 0.0;
            for (int p = max(0, c - i0); p < r; ++p) s += (double)Lb[r][p] * (double)xs[p][threadIdx.x];
            const double num = c == i ? 1.0 : -s;
            v = (float)(num / (double)Lb[r][r]);
        }
        xs[r][threadIdx.x] = v;
        x[(size_t)i * n + c] = v;
    }
}

// U[r][c] = X[n-1-r][n-1-c] for c >= r, else 0 (gptq_linalg.go:208-221).
__global__ void u_from_x_kernel(const float *__restrict__ x, float *__restrict__ u, int n) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)n * n) return;
    const int r = (int)(idx / n), c = (int)(idx - (size_t)r * n);
    u[idx] = c < r ? 0.0f : x[(size_t)(n - 1 - r) * n + (n - 1 - c)];
}

// ---- rounding ----------------------------------------------------------------

// Zero the dead columns of w [n][k] (gptq.go:643-651).
__global__ void zero_dead_kernel(float *w, int n, int k, const uint8_t *dead) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)n * k) return;
    if (dead[idx % k]) w[idx] = 0.0f;
}

// 8-bit row scales max|row| / 127 (gptq.go:675-680), NaN propagating like
// q8gemm.MaxAbs; fp32, also stored little-endian as the row's scale bytes.
__global__ __launch_bounds__(256) void row_scale_kernel(const float *__restrict__ w, int k, float *__restrict__ s) {
    __shared__ float part[4];
    __shared__ int nanp[4];
    const float *row = w + (size_t)blockIdx.x * k;
    float m = 0.0f;
    int nan = 0;
    for (int i = threadIdx.x; i < k; i += blockDim.x) {
        const float v = row[i];
        nan |= v != v;
        m = fmaxf(m, fabsf(v));
    }
    for (int off = 32; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off));
        nan |= __shfl_xor(nan, off);
    }
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6] = m;
        nanp[threadIdx.x >> 6] = nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float mm = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
        if (nanp[0] | nanp[1] | nanp[2] | nanp[3]) mm = __builtin_nanf("");
        s[blockIdx.x] = mm / 127.0f;
    }
}

__device__ __forceinline__ float f16r(float x) {
    asm volatile("" : "+v"(x));
    return (float)(_Float16)x;
}

// q4GroupScale (gptq.go:764-791) of the 32 values held one per lane by lanes
// g .. g+31 of the wavefront (the caller's x is the lane's value): peak = the
// value of largest magnitude, lowest column on ties; 16 FP16 candidates
// f16(peak / -8 * (1 - 0.02 step)); the candidate with the smallest float64
// sum of squared errors, the first on ties. Every lane returns the result.
__device__ float q4_group_scale_wave(float x, int g) {
    const int lane = threadIdx.x & 63;
    const bool in = lane >= g && lane < g + 32;
    float pv = in ? x : 0.0f;
    int pi = in ? lane : 64;
    for (int off = 1; off < 64; off <<= 1) {
        const float ov = __shfl_xor(pv, off);
        const int oi = __shfl_xor(pi, off);
        if (fabsf(ov) > fabsf(pv) || (fabsf(ov) == fabsf(pv) && oi < pi)) {
            pv = ov;
            pi = oi;
        }
    }
    const float peak = pv;  // the same on every lane
    if (peak == 0.0f) return 0.0f;
    float best = 0.0f;
    double bestErr = INFINITY;
    for (int step = 0; step < 16; ++step) {
        const float d = f16r(peak / -8.0f * (1.0f - 0.02f * (float)step));
        if (d == 0.0f) continue;
        double e = 0.0;
        if (in) {
            const float qv = fminf(7.0f, fmaxf(-8.0f, rintf(x / d)));
            const double diff = (double)x - (double)qv * (double)d;
            e = diff * diff;
        }
        for (int off = 32; off > 0; off >>= 1) e += __shfl_xor(e, off);
        if (e < bestErr) {
            best = d;
            bestErr = e;
        }
    }
    return best;
}

struct RoundArgs {
    float *w;              // [n][k], updated in place
    const float *u;        // [k][k]
    float *errs;           // [n][kRoundBlock]
    uint8_t *codes;        // 8-bit: int8 [n][k]; 4-bit: [n][k/2]
    uint8_t *scales;       // 8-bit: fp32 [n]; 4-bit: fp16 [n][k/32]
    const float *rowScale; // 8-bit row scales
    int n, k, i1, b, bits;
};

// One 128-column block of gptqRound (gptq.go:686-745): wavefront w of the
// workgroup takes weight row blockIdx.x * 8 + w; lane l holds block columns l
// and l + 64. The block's U rows sit in LDS.
__global__ __launch_bounds__(64 * kRowsPerBlock) void gptq_round_block_kernel(const RoundArgs a) {
    __shared__ float Ub[kRoundBlock][kRoundBlock + 1];
    const int b = a.b, i1 = a.i1, k = a.k;
    for (int e = threadIdx.x; e < b * b; e += blockDim.x) {
        const int p = e / b, q = e - p * b;
        Ub[p][q] = a.u[(size_t)(i1 + p) * k + i1 + q];
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (r >= a.n) return;  // whole wavefronts: the row is wave-uniform
    float *row = a.w + (size_t)r * k + i1;
    float v[2];
    int code[2] = {0, 0};
#pragma unroll
    for (int h = 0; h < 2; ++h) v[h] = lane + 64 * h < b ? row[lane + 64 * h] : 0.0f;
    float s = a.bits == 8 ? a.rowScale[r] : 0.0f;
    for (int c = 0; c < b; ++c) {
        const int slot = c >> 6, owner = c & 63;
        if (a.bits == 4 && (c & 31) == 0) {
            s = q4_group_scale_wave(slot ? v[1] : v[0], owner);
            if (lane == 0)
                ((uint16_t *)a.scales)[(size_t)r * (k / 32) + (i1 + c) / 32] =
                    __builtin_bit_cast(uint16_t, (_Float16)s);
        }
        const float lo = a.bits == 8 ? -127.0f : -8.0f, hi = a.bits == 8 ? 127.0f : 7.0f;
        // The owner lane's value, the same on every lane.
        const float wc = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, slot ? v[1] : v[0]), owner));
        const float q = s != 0.0f ? fminf(hi, fmaxf(lo, rintf(wc / s))) : 0.0f;
        const float qv = __fmul_rn(q, s);
        const float e = __fsub_rn(wc, qv) / Ub[c][c];
        if (lane == owner) {
            if (slot) {
                v[1] = qv;
                code[1] = (int)q;
            } else {
                v[0] = qv;
                code[0] = (int)q;
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int j = lane + 64 * h;
            if (j > c && j < b) v[h] = __fsub_rn(v[h], __fmul_rn(e, Ub[c][j]));
        }
        if (lane == 0) a.errs[(size_t)r * kRoundBlock + c] = e;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int j = lane + 64 * h;
        if (j < b) row[j] = v[h];
        if (a.bits == 8) {
            if (j < b) a.codes[(size_t)r * k + i1 + j] = (uint8_t)(int8_t)code[h];
        } else {
            // Byte (col/32)*16 + col%16 holds col (low nibble) and col+16
            // (high nibble), both stored plus 8.
            const int up = __shfl_down(code[h], 16);
            const int col = i1 + j;
            if (j < b && (col & 31) < 16)
                a.codes[(size_t)r * (k / 2) + (col / 32) * 16 + (col & 15)] =
                    (uint8_t)((code[h] + 8) | ((up + 8) << 4));
        }
    }
}

}  // namespace

namespace gphq {

// C [M][N] (row stride ldc) = A [M][K] . B^T for B [N][K] (row-major, strides
// lda / ldb), fp32 with fp32 sums; with accumulate, C += the product (the
// whole sum formed first and added once, as `c[i] += d[i]` after a separate
// product). The calibration pass's projections and residual adds.
int sgemm_abt(int M, int N, int K, const float *a, long lda, const float *b, long ldb, float *c, long ldc,
              bool accumulate, hipStream_t st) {
    return sgemm<0, 1>(M, N, K, 1.0f, a, lda, b, ldb, c, ldc, accumulate, false, st);
}

}  // namespace gphq

extern "C" {

int64_t gphq_gptq_work_bytes(int64_t k) {
    if (k <= 0 || k > 65536) return GPHQ_ERR_DIMENSIONS;
    return 4 * k * k + 4 * (int64_t)kPanel * k + 256;
}

int gphq_gptq_factor(const float *x_dev, int64_t rows, int64_t k, float *u_dev, uint8_t *dead_dev, void *work_dev,
                     int64_t work_bytes, void *stream) {
    if (!x_dev || !u_dev || !dead_dev || !work_dev || rows < 1 || k < 1 || k > 65536 || rows > INT32_MAX)
        return GPHQ_ERR_DIMENSIONS;
    if (work_bytes < gphq_gptq_work_bytes(k)) return GPHQ_ERR_DIMENSIONS;
    hipStream_t st = (hipStream_t)stream;
    const int n = (int)k;
    float *h = (float *)work_dev;                    // H, then X = L^-1
    float *tt = h + (size_t)n * n;                   // [64][n]
    int *bad = (int *)(tt + (size_t)kPanel * n);
    GPHQ_TRY(hip_status(hipMemsetAsync(bad, 0, sizeof(int), st)));
    // H = X^T X (gptq.go:606-622).
    GPHQ_TRY((sgemm<1, 0>(n, n, (int)rows, 1.0f, x_dev, n, x_dev, n, h, n, false, false, st)));
    hipLaunchKernelGGL(gptq_damp_kernel, dim3(1), dim3(1024), 0, st, h, n, dead_dev);
    GPHQ_TRY(launch_status());
    const size_t nn = (size_t)n * n;
    const unsigned eb = (unsigned)((nn + 255) / 256);
    // A = J H J into u_dev; lower Cholesky in place (gptq_linalg.go:68-132).
    hipLaunchKernelGGL(reverse_kernel, dim3(eb), dim3(256), 0, st, h, u_dev, n);
    GPHQ_TRY(launch_status());
    float *A = u_dev;
    for (int j0 = 0; j0 < n; j0 += kPanel) {
        const int b = std::min(kPanel, n - j0), j1 = j0 + b;
        hipLaunchKernelGGL(chol_diag_kernel, dim3(1), dim3(kPanel), 0, st, A, n, j0, b, bad);
        GPHQ_TRY(launch_status());
        if (j1 == n) break;
        hipLaunchKernelGGL(chol_panel_kernel, dim3((unsigned)((n - j1 + 255) / 256)), dim3(256), 0, st, A, n, j0, b);
        GPHQ_TRY(launch_status());
        // A22 -= L21 L21^T on the lower triangle.
        const int m = n - j1;
        GPHQ_TRY((sgemm<0, 1>(m, m, b, -1.0f, A + (size_t)j1 * n + j0, n, A + (size_t)j1 * n + j0, n,
                             A + (size_t)j1 * n + j1, n, true, true, st)));
    }
    // X = L^-1 into h (gptq_linalg.go:134-176).
    GPHQ_TRY(hip_status(hipMemsetAsync(h, 0, nn * sizeof(float), st)));
    for (int i0 = 0; i0 < n; i0 += kPanel) {
        const int b = std::min(kPanel, n - i0);
        if (i0 > 0)  // T = L[i0:i0+b][0:i0] X[0:i0][0:i0]
            GPHQ_TRY((sgemm<0, 0>(b, i0, i0, 1.0f, A + (size_t)i0 * n, n, h, n, tt, i0, false, false, st)));
        hipLaunchKernelGGL(inv_rows_kernel, dim3((unsigned)((i0 + b + 255) / 256)), dim3(256), 0, st, A, h, tt, n, i0,
                           b);
        GPHQ_TRY(launch_status());
    }
    hipLaunchKernelGGL(u_from_x_kernel, dim3(eb), dim3(256), 0, st, h, u_dev, n);
    GPHQ_TRY(launch_status());
    int flag = 0;
    GPHQ_TRY(hip_status(hipMemcpyAsync(&flag, bad, sizeof(int), hipMemcpyDeviceToHost, st)));
    GPHQ_TRY(hip_status(hipStreamSynchronize(st)));
    return flag ? GPHQ_ERR_NOT_POSITIVE_DEFINITE : GPHQ_OK;
}

int64_t gphq_gptq_round_work_bytes(int64_t n, int64_t k) {
    if (n <= 0 || k <= 0) return GPHQ_ERR_DIMENSIONS;
    return 4 * n * kRoundBlock + 4 * n;
}

int gphq_gptq_round(float *w_dev, int64_t n, int64_t k, const float *u_dev, const uint8_t *dead_dev, int bits,
                    void *codes_dev, void *scales_dev, void *work_dev, int64_t work_bytes, void *stream) {
    if (bits != 8 && bits != 4) return GPHQ_ERR_UNSUPPORTED;
    if (!w_dev || !u_dev || !dead_dev || !codes_dev || !scales_dev || !work_dev || n < 1 || k < 1 ||
        n > INT32_MAX || k > 65536 || (bits == 4 && k % 32))
        return GPHQ_ERR_DIMENSIONS;
    if (work_bytes < gphq_gptq_round_work_bytes(n, k)) return GPHQ_ERR_DIMENSIONS;
    hipStream_t st = (hipStream_t)stream;
    float *errs = (float *)work_dev;
    float *rs = errs + (size_t)n * kRoundBlock;
    const size_t nk = (size_t)n * k;
    hipLaunchKernelGGL(zero_dead_kernel, dim3((unsigned)((nk + 255) / 256)), dim3(256), 0, st, w_dev, (int)n, (int)k,
                       dead_dev);
    GPHQ_TRY(launch_status());
    if (bits == 8) {
        hipLaunchKernelGGL(row_scale_kernel, dim3((unsigned)n), dim3(256), 0, st, w_dev, (int)k, rs);
        GPHQ_TRY(launch_status());
        GPHQ_TRY(hip_status(hipMemcpyAsync(scales_dev, rs, (size_t)n * 4, hipMemcpyDeviceToDevice, st)));
    }
    RoundArgs ra{};
    ra.w = w_dev;
    ra.u = u_dev;
    ra.errs = errs;
    ra.codes = (uint8_t *)codes_dev;
    ra.scales = (uint8_t *)scales_dev;
    ra.rowScale = rs;
    ra.n = (int)n;
    ra.k = (int)k;
    ra.bits = bits;
    for (int i1 = 0; i1 < k; i1 += kRoundBlock) {
        const int b = (int)std::min<int64_t>(kRoundBlock, k - i1), i2 = i1 + b;
        ra.i1 = i1;
        ra.b = b;
        hipLaunchKernelGGL(gptq_round_block_kernel, dim3((unsigned)((n + kRowsPerBlock - 1) / kRowsPerBlock)),
                           dim3(64 * kRowsPerBlock), 0, st, ra);
        GPHQ_TRY(launch_status());
        if (i2 < k)  // W[:, i2:] -= E U[i1:i2, i2:] (gptq.go:746-760)
            GPHQ_TRY((sgemm<0, 0>((int)n, (int)(k - i2), b, -1.0f, errs, kRoundBlock, u_dev + (size_t)i1 * k + i2, k,
                                 w_dev + i2, k, true, false, st)));
    }
    return GPHQ_OK;
}

}  // extern "C"
