// Query preparation and coarse probing kernels (gfx950, wave64).
//
//   rotate        Q' = Q . R on MFMA                    (reference hybrid.cu:436-440):
//                 split-FP16 operands as dist_gemm's, or FP32
//   query_prep    k1/kb sums, ||q'||^2, Bq=8 planes     (query_kernels.cuh:73-103,117-197)
//   dist_gemm     ||q'||^2 + ||c'||^2 - 2 q'.c' on MFMA  (hybrid.cu:465-477, query_kernels.cuh:10-64):
//                 split-FP16 operands (three FP16 products per term), or FP32
//   select        per-query nprobe smallest, ascending, ties by cluster id (hybrid.cu:485-493)
//   probe_refine  exact ||q'-c'||^2 and <q',c'> of the selected probes -> g_add, g_error
//                 (query.hpp:537-545: L2 g_add = ||q'-c'||^2, IP g_add = -<q',c'>)
#include <float.h>
#include <math.h>

#include "engine_internal.h"

namespace cora {
namespace {

constexpr int kTile = 64;   // output tile per workgroup: 64 x 64
constexpr int kTileK = 16;  // K slice staged in LDS per step

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// set bits of mask below this lane
__device__ __forceinline__ uint32_t lanes_below(unsigned long long mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// C[m][n] = sum_k A[m][k] * B(k, n) on the matrix cores (v_mfma_f32_16x16x4f32: FP32
// inputs, FP32 accumulation). A is row-major [M][K]. With TRANS_B the second operand is
// Bt [N][K] (B(k, n) = Bt[n][k]) and the epilogue forms the L2 distance
// an[m] + bn[n] - 2 * C[m][n]; without it B is row-major [K][N] (the rotation Q . R).
// Four waves per workgroup, each owning a 32 x 32 quarter of the 64 x 64 tile as 2 x 2
// MFMA blocks. MFMA 16x16x4 operand layout: lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16] of the 16x4 / 4x16 blocks, and holds D[4 (l / 16) + r][l % 16],
// r = 0..3, of the 16x16 result. VEC: K % 4 == 0 and 16-byte aligned rows, loaded as
// float4; otherwise element loads (any K). Every global access is bounds-checked.
template <bool TRANS_B, bool VEC>
__global__ __launch_bounds__(256) void gemm_kernel(const float *__restrict__ A,
                                                   const float *__restrict__ B,
                                                   float *__restrict__ C, uint32_t M, uint32_t N,
                                                   uint32_t K, const float *__restrict__ an,
                                                   const float *__restrict__ bn) {
    __shared__ float As[kTileK][kTile + 4];  // [k][m]
    __shared__ float Bs[kTileK][kTile + 4];  // [k][n]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    f32x4_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // staging coordinates: 256 threads x 4 elements = one 64 x 16 slice of each operand
    const int row = tid >> 2, kq = (tid & 3) * 4;  // A and Bt: row, 4 consecutive k
    const int bk = tid >> 4, bn4 = (tid & 15) * 4;  // row-major B: k row, 4 consecutive n
    for (uint32_t k0 = 0; k0 < K; k0 += kTileK) {
        {
            const uint32_t gm = m0 + row, gk = k0 + kq;
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (gm < M) {
                const float *src = A + (size_t)gm * K + gk;
                if (VEC && gk + 4 <= K) {
                    const float4 t = *reinterpret_cast<const float4 *>(src);
                    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = gk + e < K ? src[e] : 0.0f;
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                As[kq + e][row] = v[e];
        }
        if (TRANS_B) {
            const uint32_t gn = n0 + row, gk = k0 + kq;
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (gn < N) {
                const float *src = B + (size_t)gn * K + gk;
                if (VEC && gk + 4 <= K) {
                    const float4 t = *reinterpret_cast<const float4 *>(src);
                    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = gk + e < K ? src[e] : 0.0f;
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                Bs[kq + e][row] = v[e];
        } else {
            const uint32_t gk = k0 + bk, gn = n0 + bn4;
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (gk < K) {
                const float *src = B + (size_t)gk * N + gn;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = gn + e < N ? src[e] : 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                Bs[bk][bn4 + e] = v[e];
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kTileK; kk += 4) {
            const int i = lane & 15, kl = kk + (lane >> 4);
            const float a0 = As[kl][wm + i], a1 = As[kl][wm + 16 + i];
            const float b0 = Bs[kl][wn + i], b1 = Bs[kl][wn + 16 + i];
            acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t gm = m0 + wm + 16 * ti + 4 * (lane >> 4) + r;
                const uint32_t gn = n0 + wn + 16 * tj + (lane & 15);
                if (gm < M && gn < N) {
                    float v = acc[ti][tj][r];
                    if (TRANS_B)
                        v = an[gm] + bn[gn] - 2.0f * v;
                    C[(size_t)gm * N + gn] = v;
                }
            }
}

// Distance GEMM D[m][n] = an[m] + bn[n] - 2 <A[m], Bt[n]> for the coarse probe and the
// k-means assignment, A [M][K] and Bt [N][K] row-major, K % 4 == 0, 16-byte aligned rows.
// A workgroup of four waves owns a 128 x 128 output tile, each wave a 64 x 64 quarter as
// 4 x 4 blocks of v_mfma_f32_16x16x4f32. K advances in slices of kDK (32) staged in LDS as
// [row][k] (double buffered; the next slice is loaded into registers while the current
// one is multiplied, one barrier per slice). Within each 16-wide part, MFMA j takes from lane l
// k = 4 (l / 16) + j for both operands, so each lane reads its four k values of a row
// with one 16-byte LDS read; every k meets its own partner, so the sum is the same.
constexpr int kDT = 128;  // output tile edge

template <int kDK>
__global__ __launch_bounds__(256) void dist_gemm_kernel(const float *__restrict__ A,
                                                        const float *__restrict__ Bt,
                                                        float *__restrict__ C, uint32_t M, uint32_t N,
                                                        uint32_t K, const float *__restrict__ an,
                                                        const float *__restrict__ bn) {
    constexpr int kDRow = kDK + 4;
    __shared__ __align__(16) float As[2][kDT * kDRow];
    __shared__ __align__(16) float Bs[2][kDT * kDRow];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m0 = blockIdx.y * kDT, n0 = blockIdx.x * kDT;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // staging: thread t loads rows (t >> 2) and 64 + (t >> 2) of each operand, k 4 (t & 3)
    const int srow = tid >> 2, sk = (tid & 3) * 4;
    constexpr int H = 2 * (kDK / 16);
    float4 ra[H], rb[H];
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const uint32_t gm = m0 + srow + 64 * (h & 1), gn = n0 + srow + 64 * (h & 1), gk = k0 + sk + 16 * (h >> 1);
            ra[h] = gm < M && gk < K ? *reinterpret_cast<const float4 *>(A + (size_t)gm * K + gk)
                                     : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            rb[h] = gn < N && gk < K ? *reinterpret_cast<const float4 *>(Bt + (size_t)gn * K + gk)
                                     : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int h = 0; h < H; ++h) {
            *reinterpret_cast<float4 *>(&As[buf][(srow + 64 * (h & 1)) * kDRow + sk + 16 * (h >> 1)]) = ra[h];
            *reinterpret_cast<float4 *>(&Bs[buf][(srow + 64 * (h & 1)) * kDRow + sk + 16 * (h >> 1)]) = rb[h];
        }
    };
    load(0);
    stage(0);
    __syncthreads();
    const int i16 = lane & 15, kg = (lane >> 4) * 4;
    int buf = 0;
    for (uint32_t k0 = 0; k0 < K; k0 += kDK) {
        const bool more = k0 + kDK < K;
        if (more)
            load(k0 + kDK);
#pragma unroll
        for (int ss = 0; ss < kDK / 16; ++ss) {
        float4 a[4], b[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            a[t] = *reinterpret_cast<const float4 *>(&As[buf][(wm + 16 * t + i16) * kDRow + kg + 16 * ss]);
            b[t] = *reinterpret_cast<const float4 *>(&Bs[buf][(wn + 16 * t + i16) * kDRow + kg + 16 * ss]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int ti = 0; ti < 4; ++ti) {
                const float av = j == 0 ? a[ti].x : j == 1 ? a[ti].y : j == 2 ? a[ti].z : a[ti].w;
#pragma unroll
                for (int tj = 0; tj < 4; ++tj) {
                    const float bv = j == 0 ? b[tj].x : j == 1 ? b[tj].y : j == 2 ? b[tj].z : b[tj].w;
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[ti][tj], 0, 0, 0);
                }
            }
        }
        }
        if (more) {
            stage(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }
    }
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t gm = m0 + wm + 16 * ti + 4 * (lane >> 4) + r;
            if (gm >= M)
                continue;
            const float am = an[gm];
#pragma unroll
            for (int tj = 0; tj < 4; ++tj) {
                const uint32_t gn = n0 + wn + 16 * tj + i16;
                if (gn < N)
                    C[(size_t)gm * N + gn] = am + bn[gn] - 2.0f * acc[ti][tj][r];
            }
        }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// ---- split-FP16 coarse-probe GEMM ----
//
// Each operand row x_r [P] is scaled by 2^e_r, e_r = 14 - floor(log2 max_i |x_ri|) (the
// largest magnitude lands in [2^14, 2^15), inside FP16's range), and written as two FP16
// rows hi = fp16(x 2^e), lo = fp16(x 2^e - hi) (the difference is exact in FP32), so
// x 2^e = hi + lo + d with |d| <= 2^-22 |x 2^e| (2^-25 absolute below FP16's normal range).
// The inner product is hi.hi' + hi.lo' + lo.hi' on the FP16 matrix cores with FP32
// accumulation, scaled back by 2^-(e_r + e_r'): per term a relative error of at most
// 3 * 2^-22 (the omitted lo.lo' and the two d terms), below FP32's own 24-bit rounding of
// a 768-term sum.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(64) void split_f16_kernel(const float *__restrict__ x, uint32_t rows,
                                                       uint32_t P, _Float16 *__restrict__ hi,
                                                       _Float16 *__restrict__ lo,
                                                       float *__restrict__ scale) {
    const int lane = threadIdx.x;
    for (uint32_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float *row = x + (size_t)r * P;
        float amax = 0.0f;
        for (uint32_t i = lane; i < P; i += 64)
            amax = fmaxf(amax, fabsf(row[i]));
        amax = wave_max(amax);
        // zero rows keep e = 0; the clamp keeps 2^-e a normal float
        const int e = amax > 0.0f && amax <= FLT_MAX ? min(max(14 - ilogbf(amax), -100), 100) : 0;
        for (uint32_t i = lane; i < P; i += 64) {
            const float v = ldexpf(row[i], e);
            const _Float16 h = (_Float16)v;
            hi[(size_t)r * P + i] = h;
            lo[(size_t)r * P + i] = (_Float16)(v - (float)h);
        }
        if (lane == 0)
            scale[r] = ldexpf(1.0f, -e);
    }
}

constexpr int kHT = 128;  // output tile edge
constexpr int kHK = 32;   // K per LDS stage: one v_mfma_f32_16x16x32_f16 step
constexpr int kFallbackRowTiles = 8;        // row tiles of the fused select's fallback GEMM grid
constexpr int kFallbackSelectBlocks = 512;  // workgroups of its fallback select

// LDS slot of the 8-half group g (0..3) of tile row r: the XOR spreads the 16 rows x 4
// groups of one MFMA operand read over distinct banks
__device__ __forceinline__ int hslot(int r, int g) { return r * 4 + (g ^ ((r >> 1) & 3)); }

// The coarse-probe distance of one (query, cluster) pair from the GEMM accumulator: the
// product scaled back (s is a power of two), then ||q'||^2 + ||c'||^2 - 2 <q',c'> with one
// rounding of the fused multiply-add; every mode of the GEMM forms it the same way.
__device__ __forceinline__ float probe_distance(float acc, float s, float an, float bn) {
    return __fmaf_rn(-2.0f, __fmul_rn(acc, s), __fadd_rn(an, bn));
}

// The median of three unsigned words (v_med3_u32; the compiler does not form it from min and
// max of run-time bounds): for a <= b, x clamped to [a, b].
__device__ __forceinline__ uint32_t med3_u32(uint32_t a, uint32_t b, uint32_t x) {
    uint32_t r;
    asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(x));
    return r;
}

// Fused probe select: the GEMM epilogue keeps, per query row and 128-cluster tile, the
// kSlots smallest (distance, cluster) keys (kProbeSlots, or kProbeSlotsWide for larger
// nprobe), compared on the order key with its low 7 bits
// replaced by the column in the tile (so the 128 keys of a row are distinct 32-bit values
// and the comparison is one v_med3 per slot); the exact keys of the kept columns are stored.
constexpr int kProbeSlots = 8;       // a power of two
constexpr int kProbeSlotsWide = 16;  // nprobe above 64: up to ~4.5 probes per 128-cluster tile
constexpr int kEs = kHT + 4;  // LDS row stride (floats) of the epilogue's half tile: no bank conflicts

// kMode 0: C = A . B^T (the query rotation Q . R with B = R^T). kMode 1: the distance matrix
// an[m] + bn[n] - 2 <a_m, b_n> (coarse probe). kMode 2: the same distances reduced in the
// epilogue to each row's kSlots smallest keys per 128-column tile, written to
// cand [M][ntiles][kSlots] as (order key << 32 | column) (the distance matrix is not
// written). kMode 3: distance rows of selected operand rows: output row m is A's row rmap[m],
// for m < *mcount (at most M), the grid's row tiles sweeping them mstep rows at a time.
// A [M][K] and B [N][K] are split-FP16 rows (Ah/Al, scale as; Bh/Bl, scale bs);
// K % 32 == 0, rows 16-byte aligned. 128 x 128
// output tile per workgroup of four waves (64 x 64 each, 4 x 4 MFMA blocks of 16 x 16),
// K staged in LDS 32 at a time in one buffer (the next stage's loads in registers during
// the MFMAs; 32 KB of LDS and 158 VGPRs let three workgroups share a CU, which hides the
// load latency better than two double-buffered ones). MFMA 16x16x32 operand layout: lane l
// supplies A[l % 16][8 (l / 16) .. + 7] and B[8 (l / 16) .. + 7][l % 16], and holds
// D[4 (l / 16) + r][l % 16]. Tile order: XCD x (blockIdx.x % 8) owns column tiles
// [x ncx, (x + 1) ncx), swept by groups of four row tiles, so the workgroups resident on
// an XCD share their operand tiles in its L2.
template <int kMode, int kSlots = kProbeSlots>
__global__ __launch_bounds__(256, 3) void dist_gemm_f16x3_kernel(
    const _Float16 *__restrict__ Ah, const _Float16 *__restrict__ Al, const float *__restrict__ as,
    const _Float16 *__restrict__ Bh, const _Float16 *__restrict__ Bl, const float *__restrict__ bs,
    float *__restrict__ C, uint32_t M, uint32_t N, uint32_t K, const float *__restrict__ an,
    const float *__restrict__ bn, uint32_t ncx, uint32_t mstep, const uint32_t *__restrict__ rmap,
    const uint32_t *__restrict__ mcount, unsigned long long *__restrict__ cand, uint32_t ntiles) {
    constexpr size_t kOperandBytes = 4 * kHT * 4 * sizeof(half8_t);
    constexpr size_t kHalfBytes = 64 * kEs * sizeof(float);
    constexpr size_t kLdsBytes = kMode == 2 && kHalfBytes > kOperandBytes ? kHalfBytes : kOperandBytes;
    __shared__ __align__(16) unsigned char s_raw[kLdsBytes];
    half8_t(*S)[kHT * 4] = reinterpret_cast<half8_t(*)[kHT * 4]>(s_raw);  // [Ah, Al, Bh, Bl][row x group]
    const uint32_t xcd = blockIdx.x % kNumXcd, bi = blockIdx.x / kNumXcd;
    const uint32_t grp = bi / (4 * ncx), within = bi % (4 * ncx);
    const uint32_t n0 = (xcd * ncx + within / 4) * kHT;
    const uint32_t Me = kMode == 3 ? min(M, *mcount) : M;
    if (n0 >= N)
        return;  // the whole workgroup: padding of the tile grid
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int i16 = lane & 15, g = lane >> 4;
    // staging: thread t moves group t & 3 of rows t >> 2 and 64 + (t >> 2) of each array
    const int srow = tid >> 2, sg = tid & 3;
    auto row_tile = [&](uint32_t m0) __attribute__((always_inline)) {
        f32x4_t acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        half8_t st[4][2];
        auto load = [&](uint32_t k0) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // rows past the last (M, or *mcount) repeat it: they only feed outputs that are
                // not stored; 32-bit element offsets (M K, N K < 2^31, checked by the launcher)
                const uint32_t r = min(m0 + srow + 64 * h, Me - 1);
                const uint32_t ka = (kMode == 3 ? rmap[r] : r) * K + k0 + 8 * sg;
                const uint32_t kb = min(n0 + srow + 64 * h, N - 1) * K + k0 + 8 * sg;
                st[0][h] = *reinterpret_cast<const half8_t *>(Ah + ka);
                st[1][h] = *reinterpret_cast<const half8_t *>(Al + ka);
                st[2][h] = *reinterpret_cast<const half8_t *>(Bh + kb);
                st[3][h] = *reinterpret_cast<const half8_t *>(Bl + kb);
            }
        };
        auto stage = [&]() {
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    S[a][hslot(srow + 64 * h, sg)] = st[a][h];
        };
        load(0);
        stage();
        __syncthreads();
        for (uint32_t k0 = 0; k0 < K; k0 += kHK) {
            const bool more = k0 + kHK < K;
            if (more)
                load(k0 + kHK);
            half8_t ah[4], al[4], bh[4], bl[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                ah[t] = S[0][hslot(wm + 16 * t + i16, g)];
                al[t] = S[1][hslot(wm + 16 * t + i16, g)];
                bh[t] = S[2][hslot(wn + 16 * t + i16, g)];
                bl[t] = S[3][hslot(wn + 16 * t + i16, g)];
            }
            // the three products in turn over all 16 blocks: an accumulator's dependent MFMAs
            // are 16 instructions apart
#pragma unroll
            for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                for (int tj = 0; tj < 4; ++tj)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[ti], bh[tj], acc[ti][tj], 0, 0, 0);
#pragma unroll
            for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                for (int tj = 0; tj < 4; ++tj)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[ti], bl[tj], acc[ti][tj], 0, 0, 0);
#pragma unroll
            for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                for (int tj = 0; tj < 4; ++tj)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[ti], bh[tj], acc[ti][tj], 0, 0, 0);
            if (more) {
                __syncthreads();  // every wave's operand reads of this stage are done
                stage();
                __syncthreads();
            }
        }
        if constexpr (kMode != 2) {
#pragma unroll
            for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t gm = m0 + wm + 16 * ti + 4 * g + r;
                    if (gm >= Me)
                        continue;
                    const uint32_t pm = kMode == 3 ? rmap[gm] : gm;
                    const float am = kMode != 0 ? an[pm] : 0.0f, sa = as[pm];
#pragma unroll
                    for (int tj = 0; tj < 4; ++tj) {
                        const uint32_t gn = n0 + wn + 16 * tj + i16;
                        if (gn < N)
                            C[(size_t)gm * N + gn] = kMode != 0 ? probe_distance(acc[ti][tj][r], sa * bs[gn], am, bn[gn])
                                                                : acc[ti][tj][r] * (sa * bs[gn]);
                    }
                }
        } else {
            // one half tile (64 rows x 128 columns) at a time through the LDS; four threads per
            // row each take the columns eq, eq + 4, ... and keep their kSlots smallest
            // packed keys (sorted, one v_med3 per slot and column), then the row's four
            // threads merge their lists by shuffles; thread eq stores slots eq, eq + 4, ...
            float *Et = reinterpret_cast<float *>(s_raw);
            const uint32_t tile = n0 / kHT;
            const int er = tid >> 2, eq = tid & 3;
#pragma unroll 1
            for (int h = 0; h < 2; ++h) {
                __syncthreads();  // the LDS's previous readers (operands, or the other half) are done
                if ((wave >> 1) == h) {
#pragma unroll
                    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const uint32_t gm = m0 + wm + 16 * ti + 4 * g + r;
                            const uint32_t pm = min(gm, Me - 1);
                            const float am = an[pm], sa = as[pm];
#pragma unroll
                            for (int tj = 0; tj < 4; ++tj) {
                                const uint32_t gn = min(n0 + wn + 16 * tj + i16, N - 1);
                                Et[(16 * ti + 4 * g + r) * kEs + wn + 16 * tj + i16] =
                                    probe_distance(acc[ti][tj][r], sa * bs[gn], am, bn[gn]);
                            }
                        }
                }
                __syncthreads();
                const float *erow = Et + er * kEs;
                uint32_t t[kSlots];
#pragma unroll
                for (int sl = 0; sl < kSlots; ++sl)
                    t[sl] = ~0u;
#pragma unroll 2
                for (int j = 0; j < kHT / 4; ++j) {
                    const uint32_t col = eq + 4 * j;
                    const uint32_t x = n0 + col < N ? (order_key(erow[col]) & ~127u) | col : ~0u;
#pragma unroll
                    for (int sl = kSlots - 1; sl > 0; --sl)
                        t[sl] = med3_u32(t[sl - 1], t[sl], x);
                    t[0] = min(t[0], x);
                }
#pragma unroll
                for (int o = 1; o < 4; o <<= 1) {
                    // the kSlots smallest of two sorted lists: the partner's reversed
                    // against ours gives a bitonic sequence holding them, which is then sorted
                    uint32_t p[kSlots];
#pragma unroll
                    for (int sl = 0; sl < kSlots; ++sl)
                        p[sl] = __shfl_xor(t[sl], o);
#pragma unroll
                    for (int sl = 0; sl < kSlots; ++sl)
                        t[sl] = min(t[sl], p[kSlots - 1 - sl]);
#pragma unroll
                    for (int st = kSlots / 2; st > 0; st >>= 1)
#pragma unroll
                        for (int sl = 0; sl < kSlots; ++sl)
                            if ((sl & st) == 0) {
                                const uint32_t a = t[sl], b = t[sl + st];
                                t[sl] = min(a, b);
                                t[sl + st] = max(a, b);
                            }
                }
                const uint32_t gm = m0 + h * 64 + er;
#pragma unroll
                for (int u = 0; u < kSlots / 4; ++u) {
                    const int slot = eq + 4 * u;
                    uint32_t mine = t[0];
#pragma unroll
                    for (int sl = 1; sl < kSlots; ++sl)
                        mine = sl == slot ? t[sl] : mine;
                    const uint32_t col = mine & 127u;
                    if (gm < Me)
                        cand[((size_t)gm * ntiles + tile) * kSlots + slot] =
                            n0 + col < N ? ((unsigned long long)order_key(erow[col]) << 32) | (n0 + col) : ~0ull;
                }
            }
        }
    };
    const uint32_t m_first = (grp * 4 + within % 4) * kHT;
    if constexpr (kMode != 3) {
        if (m_first < M)
            row_tile(m_first);
    } else {
        for (uint32_t m0 = m_first; m0 < Me; m0 += mstep) {
            row_tile(m0);
            if (m0 + mstep < Me)
                __syncthreads();  // the next row tile's staging overwrites the LDS
        }
    }
}

// One wave per query. Each lane owns dimensions lane + 64*i.
//
// Planes [q][16][W]: planes 0..7 hold the Bq=8 query qint = clamp(rint(q' / width))
// (reference quantize_query_bitwise_kernel, query_kernels.cuh:117-189), planes 8..15 the
// quantised residual qres = clamp(rint((q' - width*qint) / width2), -127, 127) with
// width2 = width / 254, so that width*<b,qint> + width2*<b,qres> estimates <q',b> to
// about 16 bits. The filter uses planes 0..7 only; the residual pass refines the inner
// product of surviving candidates. The residual is one fused multiply-add (the exact
// q' - width*qint rounded once), so the CPU restatement reproduces it bit for bit
// whatever the compiler's contraction setting.
__global__ __launch_bounds__(64) void query_prep_kernel(const float *__restrict__ qrot,
                                                        uint32_t P, uint32_t ex_bits,
                                                        float *__restrict__ k1,
                                                        float *__restrict__ kb,
                                                        float *__restrict__ qnorm,
                                                        float *__restrict__ qwidth,
                                                        float *__restrict__ qwidth2,
                                                        uint32_t *__restrict__ planes,
                                                        int8_t *__restrict__ qbytes) {
    const uint32_t q = blockIdx.x;
    const int lane = threadIdx.x;
    const float *row = qrot + (size_t)q * P;
    const uint32_t groups = P / 64;  // P is a multiple of 64
    float v[16];
    float sum = 0.0f, sq = 0.0f, amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        v[i] = (uint32_t)i < groups ? row[lane + 64 * i] : 0.0f;
        sum += v[i];
        sq = fmaf(v[i], v[i], sq);
        amax = fmaxf(amax, fabsf(v[i]));
    }
    sum = wave_sum(sum);
    sq = wave_sum(sq);
    amax = wave_max(amax);
    // Symmetric Bq=8 quantisation, IEEE single precision with round-half-even.
    const float width = fmaxf(amax / 127.0f, 1e-30f);
    const float inv = 1.0f / width;
    const float width2 = width / 254.0f;
    const float inv2 = 1.0f / width2;
    const uint32_t W = P / 32;
    uint32_t *out = planes + (size_t)q * 2 * kBq * W;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if ((uint32_t)i >= groups)
            break;
        int qi = (int)rintf(__fmul_rn(v[i], inv));
        qi = max(-128, min(127, qi));
        const float r = fmaf(-width, (float)qi, v[i]);
        int qr = (int)rintf(__fmul_rn(r, inv2));
        qr = max(-127, min(127, qr));
        const uint32_t u = (uint32_t)qi & 0xFFu, ur = (uint32_t)qr & 0xFFu;
        if (qbytes) {
            qbytes[(size_t)q * 2 * P + lane + 64 * i] = (int8_t)qi;
            qbytes[(size_t)q * 2 * P + P + lane + 64 * i] = (int8_t)qr;
        }
#pragma unroll
        for (int j = 0; j < kBq; ++j) {
            const unsigned long long m = __ballot((u >> j) & 1u);
            const unsigned long long mr = __ballot((ur >> j) & 1u);
            if (lane == 0) {
                out[j * W + 2 * i] = (uint32_t)m;
                out[j * W + 2 * i + 1] = (uint32_t)(m >> 32);
                out[(kBq + j) * W + 2 * i] = (uint32_t)mr;
                out[(kBq + j) * W + 2 * i + 1] = (uint32_t)(mr >> 32);
            }
        }
    }
    if (lane == 0) {
        const float cb = -(float)((1u << (ex_bits + 1)) - 1u) / 2.0f;
        k1[q] = sum * -0.5f;
        kb[q] = sum * cb;
        qnorm[q] = sq;
        qwidth[q] = width;
        qwidth2[q] = width2;
    }
}

// one wave per row, grid-stride over rows: a dispatch counts its work-items in 32 bits, so
// one workgroup per row would silently drop rows beyond 2^32 / 64 (67M rows)
// One table entry per thread: entry m of nibble group g sums, in FP32 and in dimension
// order, the components 4g + i (i = 0..3) whose bit 3 - i is set in m, starting from 0,
// then rounds to FP16 (nearest even), as precompute_lut_fp16_kernel does
// (query_kernels.cuh:199-221).
__global__ __launch_bounds__(256) void lut_build_kernel(const float *__restrict__ qrot, uint32_t P,
                                                         uint16_t *__restrict__ lut) {
    const uint32_t q = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t entries = P * 4;  // P/4 groups of 16
    if (i >= entries)
        return;
    const uint32_t g = i >> 4, m = i & 15u;
    const float *v = qrot + (size_t)q * P + 4 * g;
    float sum = 0.0f;
    if (m & 8u)
        sum += v[0];
    if (m & 4u)
        sum += v[1];
    if (m & 2u)
        sum += v[2];
    if (m & 1u)
        sum += v[3];
    lut[(size_t)q * entries + i] = __builtin_bit_cast(uint16_t, (_Float16)sum);
}

// One wave per query: e_i = width qint_i - q'_i (qint from the Bq=8 planes, two's complement),
// E+ and E- the sums of its positive and negative parts (in FP64), l1 = sum |q'_i|:
//   |Bitwise - exact| <= max(E+, E-) + 2^-24 |width ip_int| (the product's rounding),
//   |LUT4 - exact| <= (2^-11 + 2^-21) l1 + P 2^-25 (FP32 sums of up to 4 terms, rounded to
//   FP16, subnormal spacing 2^-24) + (P/8 + 1) 2^-23 l1 (the two FP32 accumulators of P/8
//   entries and their sum, with room for the entries' own rounding).
__global__ __launch_bounds__(64) void lut_margin_kernel(const float *__restrict__ qrot,
                                                         const uint32_t *__restrict__ planes,
                                                         const float *__restrict__ width, uint32_t P,
                                                         float *__restrict__ margin) {
    const uint32_t q = blockIdx.x, lane = threadIdx.x, W = P / 32;
    const float *v = qrot + (size_t)q * P;
    const uint32_t *pl = planes + (size_t)q * 2 * kBq * W;
    const double w = width[q];
    double ep = 0.0, en = 0.0, l1 = 0.0;
    for (uint32_t i = lane; i < P; i += 64) {
        int u = 0;
        for (int b = 0; b < kBq; ++b)
            u |= (int)((pl[b * W + i / 32] >> (i % 32)) & 1u) << b;
        const int qint = u >= 128 ? u - 256 : u;
        const double e = w * (double)qint - (double)v[i];
        ep += e > 0.0 ? e : 0.0;
        en += e < 0.0 ? -e : 0.0;
        l1 += fabs((double)v[i]);
    }
    for (int o = 32; o > 0; o >>= 1) {
        ep += __shfl_xor(ep, o);
        en += __shfl_xor(en, o);
        l1 += __shfl_xor(l1, o);
    }
    if (lane == 0) {
        const double u24 = 5.9604644775390625e-08;  // 2^-24
        const double d = (ep > en ? ep : en) + u24 * w * 128.0 * P +
                         (4.8828125e-04 + 4.76837158203125e-07 + (P / 8.0 + 1.0) * 2.0 * u24) * l1 +
                         P * 2.9802322387695312e-08;
        margin[q] = (float)(d * (1.0 + 1e-6)) * (1.0f + 1.0e-6f);
    }
}

__global__ __launch_bounds__(64) void row_norms_kernel(const float *__restrict__ x, uint32_t rows,
                                                       uint32_t P, float *__restrict__ out) {
    for (uint32_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float *row = x + (size_t)r * P;
        float s = 0.0f;
        for (uint32_t i = threadIdx.x; i < P; i += 64)
            s = fmaf(row[i], row[i], s);
        s = wave_sum(s);
        if (threadIdx.x == 0)
            out[r] = s;
    }
}


constexpr int kSelThreads = 256;


__device__ void block_exclusive_scan2(uint32_t &a, uint32_t &b, uint32_t *sa, uint32_t *sb,
                                      uint32_t &total_a, uint32_t &total_b) {
    const int t = threadIdx.x;
    sa[t] = a;
    sb[t] = b;
    __syncthreads();
    for (int o = 1; o < kSelThreads; o <<= 1) {
        uint32_t xa = t >= o ? sa[t - o] : 0, xb = t >= o ? sb[t - o] : 0;
        __syncthreads();
        sa[t] += xa;
        sb[t] += xb;
        __syncthreads();
    }
    total_a = sa[kSelThreads - 1];
    total_b = sb[kSelThreads - 1];
    a = sa[t] - a;
    b = sb[t] - b;
    __syncthreads();
}

constexpr uint32_t kSelLdsRow = 32768;  // rows up to this many clusters are staged in LDS (128 KB)
constexpr size_t kSelMaxDynLds = 144 * 1024;  // of the 160 KB a gfx950 workgroup may hold

// The k-th smallest order key (k >= 1) of a block's keys, each thread visiting its own
// with each_key(f). The keys first give their minimum and maximum; every pass then
// histograms the keys of the current range [lo, lo + span] into 256 bins of equal width
// (a power of two) and keeps the bin holding the k-th, narrowing the range by 8 bits, so
// keys spread over the bins even when they share their high bits. Returns the key and in
// take_eq how many keys equal to it belong to the k smallest. Block size kThreads >= 256;
// s_red holds one word per wave.
template <int kThreads, class EachKey>
__device__ uint32_t block_kth_key(EachKey each_key, uint32_t k, uint32_t *hist, uint32_t *s_red,
                                  uint32_t *s_sc, uint32_t &take_eq) {
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    constexpr uint32_t kWaves = kThreads / 64;
    uint32_t mn = 0xFFFFFFFFu, mx = 0u;
    each_key([&](uint32_t key) {
        mn = min(mn, key);
        mx = max(mx, key);
    });
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        mn = min(mn, (uint32_t)__shfl_xor(mn, o));
        mx = max(mx, (uint32_t)__shfl_xor(mx, o));
    }
    if (lane == 0) {
        s_red[wave] = mn;
        s_red[kWaves + wave] = mx;
    }
    __syncthreads();
    uint32_t lo = 0xFFFFFFFFu, hi = 0u;
    for (uint32_t w = 0; w < kWaves; ++w) {
        lo = min(lo, s_red[w]);
        hi = max(hi, s_red[kWaves + w]);
    }
    __syncthreads();
    uint32_t span = hi - lo, rem = k;
    while (span > 0) {
        const uint32_t bits = 32u - (uint32_t)__clz(span);
        const uint32_t shift = bits > 8 ? bits - 8 : 0u;
        if (t < 256)
            hist[t] = 0;
        __syncthreads();
        each_key([&](uint32_t key) {
            if (key >= lo && key - lo <= span)
                atomicAdd(&hist[(key - lo) >> shift], 1u);
        });
        __syncthreads();
        uint32_t h = t < 256 ? hist[t] : 0u, v = h;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(v, o);
            if (lane >= (uint32_t)o)
                v += y;
        }
        if (lane == 63)
            s_red[wave] = v;
        __syncthreads();
        for (uint32_t w = 0; w < wave; ++w)
            v += s_red[w];
        if (t < 256 && v >= rem && v - h < rem) {
            s_sc[0] = t;
            s_sc[1] = rem - (v - h);
        }
        __syncthreads();
        const uint32_t b = s_sc[0];
        rem = s_sc[1];
        lo += b << shift;
        span = min(span - (b << shift), (1u << shift) - 1u);
        __syncthreads();
    }
    take_eq = rem;
    return lo;
}
  // rows up to this many clusters are staged in LDS

// Per query: radix-select the key of the nprobe-th smallest distance (4 x 8-bit digits,
// each digit found by a block prefix sum over the 256-bin histogram), gather every
// smaller distance and the lowest-index ties in index order, then bitonic sort
// (key, cluster) ascending in LDS. With kLds the row's order keys are staged in LDS once.
template <bool kLds>
__device__ void select_block(const float *__restrict__ row, uint32_t nl, uint32_t k, uint32_t kpow2,
                             int32_t *__restrict__ out) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_red[2 * kSelThreads / 64], s_sc[2];
    __shared__ uint32_t sa[kSelThreads], sb[kSelThreads];
    extern __shared__ unsigned long long sel[];  // [kpow2], then the row's keys with kLds
    uint32_t *keys = reinterpret_cast<uint32_t *>(sel + kpow2);
    const uint32_t t = threadIdx.x;
    auto key_at = [&](uint32_t i) -> uint32_t {
        if constexpr (kLds)
            return keys[i];
        else
            return order_key(row[i]);
    };
    if constexpr (kLds) {
        for (uint32_t i = t; i < nl; i += kSelThreads)
            keys[i] = order_key(row[i]);
    }
    if constexpr (kLds)
        __syncthreads();
    uint32_t take_eq = 0;
    const uint32_t kth = block_kth_key<kSelThreads>(
        [&](auto f) {
            for (uint32_t i = t; i < nl; i += kSelThreads)
                f(key_at(i));
        },
        k, hist, s_red, s_sc, take_eq);
    const uint32_t chunk = (nl + kSelThreads - 1) / kSelThreads;
    const uint32_t begin = min(nl, t * chunk), end = min(nl, begin + chunk);
    uint32_t nless = 0, neq = 0;
    for (uint32_t i = begin; i < end; ++i) {
        const uint32_t key = key_at(i);
        nless += key < kth;
        neq += key == kth;
    }
    uint32_t tot_less, tot_eq;
    block_exclusive_scan2(nless, neq, sa, sb, tot_less, tot_eq);
    for (uint32_t i = begin; i < end; ++i) {
        const uint32_t key = key_at(i);
        if (key < kth) {
            sel[nless++] = ((unsigned long long)key << 32) | i;
        } else if (key == kth) {
            if (neq < take_eq)
                sel[tot_less + neq] = ((unsigned long long)key << 32) | i;
            ++neq;
        }
    }
    for (uint32_t i = k + t; i < kpow2; i += kSelThreads)
        sel[i] = ~0ull;
    __syncthreads();
    for (uint32_t size = 2; size <= kpow2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = t; i < kpow2; i += kSelThreads) {
                const uint32_t j = i ^ stride;
                if (j > i) {
                    const bool asc = (i & size) == 0;
                    const unsigned long long a = sel[i], b = sel[j];
                    if ((a > b) == asc) {
                        sel[i] = b;
                        sel[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (uint32_t i = t; i < k; i += kSelThreads)
        out[i] = (int32_t)(uint32_t)(sel[i] & 0xFFFFFFFFull);
}

template <bool kLds>
__global__ __launch_bounds__(kSelThreads) void select_kernel(const float *__restrict__ dist,
                                                             uint32_t nl, uint32_t k,
                                                             uint32_t kpow2,
                                                             int32_t *__restrict__ out) {
    select_block<kLds>(dist + (size_t)blockIdx.x * nl, nl, k, kpow2, out + (size_t)blockIdx.x * k);
}

// nlist beyond what registers hold, k <= 64: two streaming passes over the row. Each of the
// four waves owns a contiguous quarter; its lanes read 16 bytes each per step (a wave reads
// 1 KB contiguous), and each lane's keys fall into kSelGroups groups of consecutive steps.
// Pass 1 takes the groups' minima; the k-th smallest of the wave's 64 kSelGroups minima
// bounds the wave's k smallest keys (k groups hold a key at or below it). Pass 2 keeps the
// keys up to the bound (a few times k for untied data), and they are ranked by (key, index)
// within the wave and across the four waves as in select_regs_kernel. A wave keeping more
// than kSelStreamCand keys (heavy ties) sends the block to the generic selection.
constexpr uint32_t kSelGroups = 4;
constexpr uint32_t kSelStreamCand = 512;

__global__ __launch_bounds__(kSelThreads) void select_stream_kernel(const float *__restrict__ dist,
                                                                    uint32_t nl, uint32_t k,
                                                                    uint32_t kpow2,
                                                                    int32_t *__restrict__ out) {
    constexpr uint32_t kWaves = kSelThreads / 64;
    __shared__ unsigned long long s_cand[kWaves][kSelStreamCand], s_best[kWaves][64];
    __shared__ uint32_t s_over;
    const float *row = dist + (size_t)blockIdx.x * nl;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // the wave's segment, whole 256-key steps (nl % 4 == 0: 16-byte loads stay in the row)
    const uint32_t per = ((nl + kWaves * 256 - 1) / (kWaves * 256)) * 256;
    const uint32_t seg0 = min(nl, wave * per), seg1 = min(nl, seg0 + per);
    const uint32_t steps = (seg1 - seg0 + 255) / 256, gsteps = (steps + kSelGroups - 1) / kSelGroups;
    auto keys4 = [&](uint32_t j, uint32_t (&kk)[4]) {
        const uint32_t i = seg0 + j * 256 + lane * 4;
        if (i + 4 <= seg1) {
            const float4 v = *reinterpret_cast<const float4 *>(row + i);
            kk[0] = order_key(v.x);
            kk[1] = order_key(v.y);
            kk[2] = order_key(v.z);
            kk[3] = order_key(v.w);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                kk[e] = i + e < seg1 ? order_key(row[i + e]) : 0xFFFFFFFFu;
        }
    };
    uint32_t gm[kSelGroups];
#pragma unroll
    for (uint32_t g = 0; g < kSelGroups; ++g)
        gm[g] = 0xFFFFFFFFu;
    for (uint32_t j = 0; j < steps; ++j) {
        uint32_t kk[4];
        keys4(j, kk);
        const uint32_t g = j / gsteps;
        const uint32_t m = min(min(kk[0], kk[1]), min(kk[2], kk[3]));
#pragma unroll
        for (uint32_t x = 0; x < kSelGroups; ++x)
            if (x == g)
                gm[x] = min(gm[x], m);
    }
    // k-th smallest of the wave's 64 * kSelGroups group minima (ties by lane, then group)
    uint32_t rk[kSelGroups];
#pragma unroll
    for (uint32_t x = 0; x < kSelGroups; ++x)
        rk[x] = 0;
    for (int src = 0; src < 64; ++src) {
#pragma unroll
        for (uint32_t y = 0; y < kSelGroups; ++y) {
            const uint32_t o = (uint32_t)__shfl((int)gm[y], src), oi = (uint32_t)src * kSelGroups + y;
#pragma unroll
            for (uint32_t x = 0; x < kSelGroups; ++x)
                rk[x] += (o < gm[x] || (o == gm[x] && oi < lane * kSelGroups + x)) ? 1u : 0u;
        }
    }
    uint32_t bound = 0xFFFFFFFFu;  // set by the one minimum of rank k - 1
#pragma unroll
    for (uint32_t x = 0; x < kSelGroups; ++x) {
        const unsigned long long bm = __ballot(rk[x] == k - 1);
        if (bm)
            bound = (uint32_t)__shfl((int)gm[x], __ffsll((long long)bm) - 1);
    }
    if (t == 0)
        s_over = 0;
    uint32_t c = 0;
    for (uint32_t j = 0; j < steps; ++j) {
        uint32_t kk[4];
        keys4(j, kk);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t i = seg0 + j * 256 + lane * 4 + e;
            const bool take = i < seg1 && kk[e] <= bound;
            const unsigned long long tm = __ballot(take);
            const uint32_t pos = c + lanes_below(tm);
            if (take && pos < kSelStreamCand)
                s_cand[wave][pos] = ((unsigned long long)kk[e] << 32) | i;
            c += (uint32_t)__popcll(tm);
        }
    }
    __syncthreads();  // s_over cleared before any wave sets it
    if (c > kSelStreamCand && lane == 0)
        s_over = 1;
    __syncthreads();
    if (s_over) {
        select_block<false>(dist + (size_t)blockIdx.x * nl, nl, k, kpow2, out + (size_t)blockIdx.x * k);
        return;
    }
    for (uint32_t e = lane; e < c; e += 64) {
        const unsigned long long v = s_cand[wave][e];
        uint32_t rk = 0;
        for (uint32_t f = 0; f < c; ++f)
            rk += s_cand[wave][f] < v ? 1u : 0u;
        if (rk < k)
            s_best[wave][rk] = v;
    }
    for (uint32_t r = c + lane; r < k; r += 64)
        s_best[wave][r] = ~0ull;  // a segment with fewer than k keys
    __syncthreads();
    for (uint32_t i = t; i < kWaves * k; i += kSelThreads) {
        const uint32_t w = i / k;
        const unsigned long long v = s_best[w][i % k];
        if (v == ~0ull)
            continue;
        uint32_t rk = i % k;
        for (uint32_t w2 = 0; w2 < kWaves; ++w2) {
            if (w2 == w)
                continue;
            uint32_t lo = 0, hi = k;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (s_best[w2][mid] < v)
                    lo = mid + 1;
                else
                    hi = mid;
            }
            rk += lo;
        }
        if (rk < k)
            out[(size_t)blockIdx.x * k + rk] = (int32_t)(uint32_t)(v & 0xFFFFFFFFull);
    }
}

// Fused probe select, second half: per query (one wave of four per workgroup) the k smallest
// of the candidate keys that the distance GEMM kept, kProbeSlots per 128-cluster tile, each
// (order key << 32 | cluster), so ties fall to the lower cluster id as in the other selects.
// The k-th smallest of the 64 lanes' minima (the first keys of each lane's tiles) bounds the
// k-th smallest key, since k distinct keys lie at or below it; the keys up to the bound are
// compacted in LDS and ranked exactly by counting. The result is proven when no tile can have
// dropped a key of it: a tile dropped only columns whose packed comparison key, the order key
// with its low 7 bits cleared, is at least that of its last kept key, so a tile whose last
// key, so truncated, lies above the k-th key's order key dropped nothing that belongs. A query
// that fails this (kProbeSlots of its nearest clusters in one tile, or ties within 128 ulps of the
// k-th distance), or that has more than kMergeCap keys below the bound, goes to the fallback
// list: its distance row is computed again and selected by the generic select.
// A lane holds all kProbeSlots keys of its tiles (lane + 64 i, i < kMergeTiles: up to 512
// tiles, nlist 65,536) in registers, read once as whole 64-byte tile records; the bound, the
// compaction and the proof all work from them (three passes over the candidates in memory
// fetched them three times from HBM at nlist 65,536: 0.98 GB for 0.33 GB of keys; select and
// g_add 0.57 -> 0.53 ms at config 5).
constexpr uint32_t kMergeWaves = 4;
constexpr uint32_t kMergeCap = 1024;
constexpr uint32_t kMergeTiles = 8;

__global__ __launch_bounds__(64 * kMergeWaves) void probe_merge_kernel(
    const unsigned long long *__restrict__ cand, uint32_t nq, uint32_t ntiles, uint32_t k,
    int32_t *__restrict__ idx, uint32_t *__restrict__ fb_count, uint32_t *__restrict__ fb_rows) {
    __shared__ unsigned long long s_c[kMergeWaves][kMergeCap];
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t q = blockIdx.x * kMergeWaves + w;
    const bool live = q < nq;  // a wave past the last query still meets every barrier
    const unsigned long long *cq = cand + (size_t)(live ? q : 0) * ntiles * kProbeSlots;
    static_assert(kProbeSlots == 8, "a tile's keys are one 64-byte record");
    unsigned long long keys[kMergeTiles][kProbeSlots];
#pragma unroll
    for (uint32_t i = 0; i < kMergeTiles; ++i) {
        const uint32_t t = lane + 64 * i;
        if (live && t < ntiles) {
            const uint4 *rec = reinterpret_cast<const uint4 *>(cq + (size_t)t * kProbeSlots);
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint4 v = rec[h];
                keys[i][2 * h] = ((unsigned long long)v.y << 32) | v.x;
                keys[i][2 * h + 1] = ((unsigned long long)v.w << 32) | v.z;
            }
        } else {
#pragma unroll
            for (int sl = 0; sl < kProbeSlots; ++sl)
                keys[i][sl] = ~0ull;
        }
    }
    unsigned long long m = ~0ull;
#pragma unroll
    for (uint32_t i = 0; i < kMergeTiles; ++i)
        m = min(m, keys[i][0]);
    // bitonic sort of the 64 lane minima, ascending by lane
    for (uint32_t size = 2; size <= 64; size <<= 1)
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            const unsigned long long o = ((unsigned long long)(uint32_t)__shfl_xor((int)(uint32_t)(m >> 32), (int)stride) << 32) |
                                         (uint32_t)__shfl_xor((int)(uint32_t)m, (int)stride);
            const bool take_min = ((lane & stride) == 0) == ((lane & size) == 0);
            m = take_min ? min(m, o) : max(m, o);
        }
    const unsigned long long bound =
        ((unsigned long long)(uint32_t)__shfl((int)(uint32_t)(m >> 32), (int)(k - 1)) << 32) |
        (uint32_t)__shfl((int)(uint32_t)m, (int)(k - 1));
    uint32_t cnt = 0;
    if (live)
#pragma unroll
        for (uint32_t i = 0; i < kMergeTiles; ++i) {
#pragma unroll
            for (int sl = 0; sl < kProbeSlots; ++sl) {
                const unsigned long long key = keys[i][sl];
                const bool take = key <= bound && key != ~0ull;
                const unsigned long long tm = __ballot(take);
                const uint32_t pos = cnt + lanes_below(tm);
                if (take && pos < kMergeCap)
                    s_c[w][pos] = key;
                cnt += (uint32_t)__popcll(tm);
            }
        }
    __syncthreads();
    bool fallback = cnt > kMergeCap;
    if (live && !fallback) {
        unsigned long long kth = 0;
        for (uint32_t i0 = 0; i0 < cnt; i0 += 64) {
            const uint32_t i = i0 + lane;
            const unsigned long long key = i < cnt ? s_c[w][i] : ~0ull;
            uint32_t r = 0;
            for (uint32_t j = 0; j < cnt; ++j)
                r += s_c[w][j] < key;
            if (i < cnt && r < k)
                idx[(size_t)q * k + r] = (int32_t)(uint32_t)key;
            if (i < cnt && r == k - 1)
                kth = key;
        }
        // one lane holds the k-th key (cnt >= k: k keys lie at or below the bound)
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            kth = max(kth, ((unsigned long long)(uint32_t)__shfl_xor((int)(uint32_t)(kth >> 32), o) << 32) |
                               (uint32_t)__shfl_xor((int)(uint32_t)kth, o));
        const uint32_t kth_key = (uint32_t)(kth >> 32);
        bool open = false;
#pragma unroll
        for (uint32_t i = 0; i < kMergeTiles; ++i) {
            const unsigned long long last = keys[i][kProbeSlots - 1];
            open |= last != ~0ull && ((uint32_t)(last >> 32) & ~127u) <= kth_key;
        }
        fallback = __ballot(open) != 0;
    }
    if (live && fallback && lane == 0)
        fb_rows[atomicAdd(fb_count, 1u)] = q;
}

// Fused probe select, second half for nprobe above 64 (kProbeSlotsWide keys per tile), one
// workgroup per query. The k-th smallest order key T among the candidates is found bit by bit
// from the top (each step counts the keys at or below a trial value over the workgroup; the
// order keys are held in registers, 32 a thread); every candidate whose order key is at most
// T (k of them, plus the ties of T) is compacted into LDS and sorted by (order key, cluster),
// and the first k are the result, ties falling to the lower cluster id. The proof and the
// fallback are those of probe_merge_kernel: more than kMergeBigCap keys at or below T, or a
// tile whose last kept key, truncated, lies at or below T, send the query to the fallback list.
constexpr uint32_t kMergeBigThreads = 256;
constexpr uint32_t kMergeBigPer = 32;  // candidate keys per thread: 512 tiles x 16 slots
constexpr uint32_t kMergeBigCap = 2048;
constexpr uint32_t kMergeBigMaxProbe = 1024;

template <int kSlots>
__global__ __launch_bounds__(kMergeBigThreads) void probe_merge_big_kernel(
    const unsigned long long *__restrict__ cand, uint32_t nq, uint32_t ntiles, uint32_t k,
    int32_t *__restrict__ idx, uint32_t *__restrict__ fb_count, uint32_t *__restrict__ fb_rows) {
    __shared__ unsigned long long s_sel[kMergeBigCap];
    __shared__ uint32_t s_red[2][kMergeBigThreads / 64];
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t q = blockIdx.x;
    const unsigned long long *cq = cand + (size_t)q * ntiles * kSlots;
    const uint32_t n = ntiles * kSlots;  // <= kMergeBigPer * kMergeBigThreads (checked by the launcher)
    uint32_t hk[kMergeBigPer];
#pragma unroll
    for (uint32_t r = 0; r < kMergeBigPer; ++r) {
        const uint32_t i = r * kMergeBigThreads + t;
        hk[r] = i < n ? (uint32_t)(cq[i] >> 32) : ~0u;  // an empty slot's key is ~0
    }
    // the workgroup's count of keys at or below x (one barrier; the two halves of s_red
    // alternate between consecutive calls)
    uint32_t parity = 0;
    auto count_le = [&](uint32_t x, bool strict) -> uint32_t {
        uint32_t c = 0;
#pragma unroll
        for (uint32_t r = 0; r < kMergeBigPer; ++r)
            c += hk[r] != ~0u && (strict ? hk[r] < x : hk[r] <= x) ? 1u : 0u;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            c += __shfl_xor(c, o);
        if (lane == 0)
            s_red[parity][wave] = c;
        __syncthreads();
        uint32_t all = 0;
#pragma unroll
        for (uint32_t w = 0; w < kMergeBigThreads / 64; ++w)
            all += s_red[parity][w];
        parity ^= 1u;
        return all;
    };
    uint32_t T = 0;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t trial = T | ((1u << bit) - 1u);
        if (count_le(trial, false) < k)
            T |= 1u << bit;
    }
    const uint32_t n_le = count_le(T, false);
    bool fallback = n_le > kMergeBigCap;
    if (!fallback) {
        // compact the keys at or below T (thread order), then sort them
        uint32_t mine = 0;
#pragma unroll
        for (uint32_t r = 0; r < kMergeBigPer; ++r)
            mine += hk[r] != ~0u && hk[r] <= T ? 1u : 0u;
        uint32_t x = mine;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(x, o);
            if (lane >= (uint32_t)o)
                x += y;
        }
        if (lane == 63)
            s_red[parity][wave] = x;
        __syncthreads();
        uint32_t pos = x - mine;
        for (uint32_t w = 0; w < wave; ++w)
            pos += s_red[parity][w];
#pragma unroll
        for (uint32_t r = 0; r < kMergeBigPer; ++r) {
            const uint32_t i = r * kMergeBigThreads + t;
            if (hk[r] != ~0u && hk[r] <= T) {
                const unsigned long long key = cq[i];
                s_sel[pos++] = (key & 0xFFFFFFFF00000000ull) | (uint32_t)key;
            }
        }
        uint32_t m = 1;
        while (m < n_le)
            m <<= 1;
        for (uint32_t i = n_le + t; i < m; i += kMergeBigThreads)
            s_sel[i] = ~0ull;
        __syncthreads();
        for (uint32_t size = 2; size <= m; size <<= 1)
            for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                for (uint32_t i = t; i < m; i += kMergeBigThreads) {
                    const uint32_t j = i ^ stride;
                    if (j > i) {
                        const bool asc = (i & size) == 0;
                        const unsigned long long a = s_sel[i], b = s_sel[j];
                        if ((a > b) == asc) {
                            s_sel[i] = b;
                            s_sel[j] = a;
                        }
                    }
                }
                __syncthreads();
            }
        // proven unless a tile dropped a column whose truncated key is at most the k-th's
        const uint32_t kth_key = (uint32_t)(s_sel[k - 1] >> 32);
        bool open = false;
        for (uint32_t tl = t; tl < ntiles; tl += kMergeBigThreads) {
            const unsigned long long last = cq[(size_t)tl * kSlots + kSlots - 1];
            open |= last != ~0ull && ((uint32_t)(last >> 32) & ~127u) <= kth_key;
        }
        fallback = __syncthreads_or(open) != 0;
        if (!fallback)
            for (uint32_t i = t; i < k; i += kMergeBigThreads)
                idx[(size_t)q * k + i] = (int32_t)(uint32_t)(s_sel[i] & 0xFFFFFFFFull);
    }
    if (fallback && t == 0)
        fb_rows[atomicAdd(fb_count, 1u)] = q;
    (void)nq;
}

// The fallback rows of the fused select: row r of dist (the distances of query rows[r],
// computed again) through the generic block select, rows swept by the grid.
__global__ __launch_bounds__(kSelThreads) void select_rows_kernel(const float *__restrict__ dist, uint32_t nl,
                                                                  uint32_t k, uint32_t kpow2,
                                                                  const uint32_t *__restrict__ rows,
                                                                  const uint32_t *__restrict__ count,
                                                                  int32_t *__restrict__ out) {
    const uint32_t n = *count;
    for (uint32_t r = blockIdx.x; r < n; r += gridDim.x) {
        select_block<false>(dist + (size_t)r * nl, nl, k, kpow2, out + (size_t)rows[r] * k);
        __syncthreads();  // the next row reuses the LDS
    }
}

// One wave per query (four per workgroup), no workgroup barriers: the k-th smallest order
// key by range narrowing (a min/max pass, then passes that histogram the keys of the
// current range into 256 equal power-of-two bins held in the wave's LDS and keep the bin
// holding the k-th), then every smaller key and the lowest-index ties in index order
// (ballot compaction), then a bitonic sort of the kpow2 slots in the wave's LDS. The row
// is read once from HBM and the later passes hit L2.
constexpr int kSelWaveThreads = 256;
constexpr uint32_t kSelWaveMaxK = 1024;  // kpow2 limit (8 KB of LDS per wave)

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

__global__ __launch_bounds__(kSelWaveThreads) void select_wave_kernel(const float *__restrict__ dist,
                                                                      uint32_t nq, uint32_t nl, uint32_t k,
                                                                      uint32_t kpow2,
                                                                      int32_t *__restrict__ out) {
    extern __shared__ unsigned long long s_sel_all[];  // [4 waves][kpow2]
    __shared__ uint32_t s_hist_all[kSelWaveThreads / 64][256];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = blockIdx.x * (kSelWaveThreads / 64) + wave;
    if (q >= nq)
        return;  // whole wave: no barrier below involves other waves
    unsigned long long *sel = s_sel_all + (size_t)wave * kpow2;
    uint32_t *hist = s_hist_all[wave];
    const float *row = dist + (size_t)q * nl;
    // keys visited 4 per lane per load (float4 when the row is 16-byte aligned), four
    // loads in flight per lane: chunk c of the row is indices [256 c, 256 c + 256), lane l
    // holding [256 c + 4 l, 256 c + 4 l + 4)
    const bool vec = (nl & 3u) == 0;
    const uint32_t nchunks = (nl + 255) / 256;
    auto load4 = [&](uint32_t c, uint32_t (&key)[4]) {
        const uint32_t i = 256 * c + 4 * lane;
        if (vec && i + 4 <= nl) {
            const float4 v = *reinterpret_cast<const float4 *>(row + i);
            key[0] = order_key(v.x);
            key[1] = order_key(v.y);
            key[2] = order_key(v.z);
            key[3] = order_key(v.w);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                key[j] = i + j < nl ? order_key(row[i + j]) : 0xFFFFFFFFu;
        }
    };
    // f(key, index) for every key of the row (index >= nl marks padding)
    auto each = [&](auto f) {
        uint32_t c = 0;
        for (; c + 4 <= nchunks; c += 4) {
            uint32_t key[4][4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                load4(c + u, key[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    f(key[u][j], 256 * (c + u) + 4 * lane + j);
        }
        for (; c < nchunks; ++c) {
            uint32_t key[4];
            load4(c, key);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                f(key[j], 256 * c + 4 * lane + j);
        }
    };
    uint32_t mn = 0xFFFFFFFFu, mx = 0u;
    each([&](uint32_t key, uint32_t i) {
        if (i < nl) {
            mn = min(mn, key);
            mx = max(mx, key);
        }
    });
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        mn = min(mn, (uint32_t)__shfl_xor(mn, o));
        mx = max(mx, (uint32_t)__shfl_xor(mx, o));
    }
    uint32_t lo = mn, span = mx - mn, rem = k;
    while (span > 0) {
        const uint32_t bits = 32u - (uint32_t)__clz(span);
        const uint32_t shift = bits > 8 ? bits - 8 : 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            hist[4 * lane + j] = 0;
        wave_sync();
        each([&](uint32_t key, uint32_t i) {
            if (i < nl && key >= lo && key - lo <= span)
                atomicAdd(&hist[(key - lo) >> shift], 1u);
        });
        wave_sync();
        uint32_t h[4], sum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h[j] = hist[4 * lane + j];
            sum += h[j];
        }
        uint32_t incl = sum;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(incl, o);
            if (lane >= (uint32_t)o)
                incl += y;
        }
        const uint32_t before = incl - sum;
        const unsigned long long m = __ballot(before < rem && incl >= rem);
        const uint32_t src = (uint32_t)__ffsll((long long)m) - 1u;
        uint32_t b = 0, r2 = 0;
        if (lane == src) {
            uint32_t c = before;
            int j = 0;
            while (j < 3 && c + h[j] < rem) {
                c += h[j];
                ++j;
            }
            b = 4 * lane + (uint32_t)j;
            r2 = rem - c;
        }
        b = __shfl(b, (int)src);
        rem = __shfl(r2, (int)src);
        lo += b << shift;
        span = min(span - (b << shift), (1u << shift) - 1u);
        wave_sync();
    }
    const uint32_t kth = lo, take_eq = rem, strict_total = k - take_eq;
    // gather in index order: per chunk, lane l's keys precede lane l + 1's
    uint32_t n_less = 0, n_eq = 0;
    for (uint32_t c = 0; c < nchunks; ++c) {
        uint32_t key[4];
        load4(c, key);
        uint32_t cl = 0, ce = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool valid = 256 * c + 4 * lane + j < nl;
            cl += valid && key[j] < kth;
            ce += valid && key[j] == kth;
        }
        uint32_t il = cl, ie = ce;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t yl = __shfl_up(il, o), ye = __shfl_up(ie, o);
            if (lane >= (uint32_t)o) {
                il += yl;
                ie += ye;
            }
        }
        uint32_t pl = n_less + il - cl, pe = n_eq + ie - ce;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t i = 256 * c + 4 * lane + j;
            if (i < nl && key[j] < kth) {
                sel[pl++] = ((unsigned long long)key[j] << 32) | i;
            } else if (i < nl && key[j] == kth) {
                if (pe < take_eq)
                    sel[strict_total + pe] = ((unsigned long long)key[j] << 32) | i;
                ++pe;
            }
        }
        n_less += __shfl(il, 63);
        n_eq += __shfl(ie, 63);
    }
    for (uint32_t i = k + lane; i < kpow2; i += 64)
        sel[i] = ~0ull;
    wave_sync();
    for (uint32_t size = 2; size <= kpow2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = lane; i < kpow2; i += 64) {
                const uint32_t j = i ^ stride;
                if (j > i) {
                    const bool asc = (i & size) == 0;
                    const unsigned long long a = sel[i], c = sel[j];
                    if ((a > c) == asc) {
                        sel[i] = c;
                        sel[j] = a;
                    }
                }
            }
            wave_sync();
        }
    }
    for (uint32_t i = lane; i < k; i += 64)
        out[(size_t)q * k + i] = (int32_t)(uint32_t)(sel[i] & 0xFFFFFFFFull);
}

// Large nlist: one block of 1,024 threads per query, thread t holding the order keys of
// clusters [t * R, t * R + R) in registers (nl <= 1024 * R), so the row is read once.
// Same selection as select_kernel: radix select of the nprobe-th key, every smaller key
// plus the lowest-index ties in index order, bitonic sort in LDS.
constexpr int kSelBigThreads = 1024;

constexpr uint32_t kSelCand = 256;  // per-wave candidates of the fast path

template <int R, int kThreads = kSelBigThreads>
__global__ __launch_bounds__(kThreads) void select_regs_kernel(const float *__restrict__ dist,
                                                               uint32_t nl, uint32_t k,
                                                               uint32_t kpow2,
                                                               int32_t *__restrict__ out) {
    constexpr uint32_t kWaves = kThreads / 64;
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_red[2 * kThreads / 64], s_sc[2];
    __shared__ unsigned long long s_cand[kWaves][kSelCand], s_best[kWaves][64];
    __shared__ uint32_t s_over;
    extern __shared__ unsigned long long sel[];  // [kpow2]
    const float *row = dist + (size_t)blockIdx.x * nl;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t begin = t * R;
    uint32_t key[R];
    if (R % 4 == 0 && (nl & 3u) == 0 && begin + R <= nl) {
#pragma unroll
        for (int r = 0; r < R; r += 4) {  // the thread's R keys as 16-byte loads
            const float4 v = *reinterpret_cast<const float4 *>(row + begin + r);
            key[r] = order_key(v.x);
            key[r + 1] = order_key(v.y);
            key[r + 2] = order_key(v.z);
            key[r + 3] = order_key(v.w);
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r)
            key[r] = begin + r < nl ? order_key(row[begin + r]) : 0xFFFFFFFFu;
    }
    // inclusive block scan over the block (s_red: one word per wave)
    auto incl_scan = [&](uint32_t v) -> uint32_t {
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(v, o);
            if (lane >= (uint32_t)o)
                v += y;
        }
        if (lane == 63)
            s_red[wave] = v;
        __syncthreads();
        uint32_t add = 0;
        for (uint32_t w = 0; w < wave; ++w)
            add += s_red[w];
        __syncthreads();
        return v + add;
    };
    // k <= 64: each wave keeps the keys of its segment up to the k-th smallest of its 64
    // lane minima (k lanes hold a key at or below it, so the wave's k smallest keys are all
    // kept; a few times k keys for untied data), ranks them by (key, index) within the wave,
    // and the block ranks the waves' sorted k best against each other by binary search (two
    // barriers in all). A wave keeping more than kSelCand keys (heavy ties) sends the block
    // to the radix selection below.
    if (k <= 64) {
        uint32_t m = 0xFFFFFFFFu;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (begin + r < nl)
                m = min(m, key[r]);
        uint32_t mrank = 0;  // rank of this lane's minimum among the wave's (ties by lane)
        for (int j = 0; j < 64; ++j) {
            const uint32_t o = (uint32_t)__shfl((int)m, j);
            mrank += (o < m || (o == m && (uint32_t)j < lane)) ? 1u : 0u;
        }
        const unsigned long long bm = __ballot(mrank == k - 1);
        const uint32_t bound = (uint32_t)__shfl((int)m, __ffsll((long long)bm) - 1);
        if (t == 0)
            s_over = 0;
        uint32_t c = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool take = begin + r < nl && key[r] <= bound;
            const unsigned long long tm = __ballot(take);
            const uint32_t pos = c + lanes_below(tm);
            if (take && pos < kSelCand)
                s_cand[wave][pos] = ((unsigned long long)key[r] << 32) | (begin + r);
            c += (uint32_t)__popcll(tm);
        }
        __syncthreads();  // s_over cleared before any wave sets it
        if (c > kSelCand && lane == 0)
            s_over = 1;
        __syncthreads();
        if (!s_over) {
            for (uint32_t e = lane; e < c; e += 64) {
                const unsigned long long v = s_cand[wave][e];
                uint32_t rk = 0;
                for (uint32_t f = 0; f < c; ++f)
                    rk += s_cand[wave][f] < v ? 1u : 0u;
                if (rk < k)
                    s_best[wave][rk] = v;
            }
            for (uint32_t r = c + lane; r < k; r += 64)
                s_best[wave][r] = ~0ull;  // a segment with fewer than k keys
            __syncthreads();
            for (uint32_t i = t; i < kWaves * k; i += kThreads) {
                const uint32_t w = i / k;
                const unsigned long long v = s_best[w][i % k];
                if (v == ~0ull)
                    continue;
                uint32_t rk = i % k;
                for (uint32_t w2 = 0; w2 < kWaves; ++w2) {
                    if (w2 == w)
                        continue;
                    uint32_t lo = 0, hi = k;  // entries of the sorted list w2 below v
                    while (lo < hi) {
                        const uint32_t mid = (lo + hi) >> 1;
                        if (s_best[w2][mid] < v)
                            lo = mid + 1;
                        else
                            hi = mid;
                    }
                    rk += lo;
                }
                if (rk < k)
                    out[(size_t)blockIdx.x * k + rk] = (int32_t)(uint32_t)(v & 0xFFFFFFFFull);
            }
            return;
        }
    }
    uint32_t take_eq = 0;
    const uint32_t kth = block_kth_key<kThreads>(
        [&](auto f) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (begin + r < nl)
                    f(key[r]);
        },
        k, hist, s_red, s_sc, take_eq);
    uint32_t nless = 0, neq = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (begin + r < nl) {
            nless += key[r] < kth;
            neq += key[r] == kth;
        }
    }
    // exclusive prefixes of both counts in index order; the keys below kth number
    // k - take_eq, so the ties are placed after them
    const uint32_t less_before = incl_scan(nless) - nless;
    const uint32_t eq_before = incl_scan(neq) - neq;
    const uint32_t strict_total = k - take_eq;
    uint32_t nl_i = less_before, ne_i = eq_before;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (begin + r < nl) {
            if (key[r] < kth) {
                sel[nl_i++] = ((unsigned long long)key[r] << 32) | (begin + r);
            } else if (key[r] == kth) {
                if (ne_i < take_eq)
                    sel[strict_total + ne_i] = ((unsigned long long)key[r] << 32) | (begin + r);
                ++ne_i;
            }
        }
    }
    for (uint32_t i = k + t; i < kpow2; i += kThreads)
        sel[i] = ~0ull;
    __syncthreads();
    for (uint32_t size = 2; size <= kpow2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = t; i < kpow2; i += kThreads) {
                const uint32_t j = i ^ stride;
                if (j > i) {
                    const bool asc = (i & size) == 0;
                    const unsigned long long a = sel[i], b = sel[j];
                    if ((a > b) == asc) {
                        sel[i] = b;
                        sel[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (uint32_t i = t; i < k; i += kThreads)
        out[(size_t)blockIdx.x * k + i] = (int32_t)(uint32_t)(sel[i] & 0xFFFFFFFFull);
}

// 4 blocks of 256 threads a CU, on 256 CUs
constexpr uint32_t kRefineGrid = 1024;

// A block (4 waves) per query, over a grid of at most kRefineGrid blocks that strides
// through the queries: once its blocks are dispatched, the hardware places the workgroups of
// the pair scheduling, which runs beside this kernel on another stream, in the wave slots left
// free (with a block per query it would hand every freed slot back to this kernel and the
// scheduling would wait for its end). Each wave takes probes p = wave, wave + 4, ..., two
// at a time with both centroid rows' loads issued together.
__global__ __launch_bounds__(256) void probe_refine_kernel(const float *__restrict__ qrot,
                                                           const float *__restrict__ cent,
                                                           const int32_t *__restrict__ idx,
                                                           uint32_t nprobe, uint32_t P, int metric,
                                                           float *__restrict__ gadd,
                                                           float *__restrict__ gerr,
                                                           float err_scale, uint32_t nq) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t groups = P / 64;
    for (uint32_t q = blockIdx.x; q < nq; q += gridDim.x) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = (uint32_t)i < groups ? qrot[(size_t)q * P + lane + 64 * i] : 0.0f;
        for (uint32_t p0 = wave; p0 < nprobe; p0 += 8) {
            const bool two = p0 + 4 < nprobe;
            const float *crow[2];
            crow[0] = cent + (size_t)idx[(size_t)q * nprobe + p0] * P;
            crow[1] = cent + (size_t)idx[(size_t)q * nprobe + (two ? p0 + 4 : p0)] * P;
            float cv[2][16];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    cv[h][i] = (uint32_t)i < groups ? crow[h][lane + 64 * i] : 0.0f;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (h == 1 && !two)
                    break;
                float l2 = 0.0f, ip = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    if ((uint32_t)i >= groups)
                        break;
                    const float d = v[i] - cv[h][i];
                    l2 = fmaf(d, d, l2);
                    ip = fmaf(v[i], cv[h][i], ip);
                }
                l2 = wave_sum(l2);
                ip = wave_sum(ip);
                const uint32_t p = p0 + 4 * h;
                if (lane == 0) {
                    gadd[(size_t)q * nprobe + p] = metric == 0 ? l2 : -ip;
                    gerr[(size_t)q * nprobe + p] = err_scale * sqrtf(fmaxf(l2, 0.0f));
                }
            }
        }
    }
}

}  // namespace

void launch_rotate(const float *q, const float *R, float *out, uint32_t nq, uint32_t dim,
                   uint32_t P, hipStream_t s) {
    dim3 grid((P + kTile - 1) / kTile, (nq + kTile - 1) / kTile);
    gemm_kernel<false, false><<<grid, 256, 0, s>>>(q, R, out, nq, P, dim, nullptr, nullptr);
}

void launch_query_prep(const float *qrot, uint32_t nq, uint32_t P, uint32_t ex_bits, float *k1,
                       float *kb, float *qnorm, float *qwidth, float *qwidth2, uint32_t *qplanes,
                       int8_t *qbytes, hipStream_t s) {
    query_prep_kernel<<<nq, 64, 0, s>>>(qrot, P, ex_bits, k1, kb, qnorm, qwidth, qwidth2, qplanes, qbytes);
}

void launch_lut_margin(const float *qrot, const uint32_t *planes, const float *width, uint32_t nq, uint32_t P,
                       float *margin, hipStream_t s) {
    if (nq)
        lut_margin_kernel<<<nq, 64, 0, s>>>(qrot, planes, width, P, margin);
}

void launch_lut_build(const float *qrot, uint32_t nq, uint32_t P, uint16_t *lut, hipStream_t s) {
    if (nq)
        lut_build_kernel<<<dim3((P * 4 + 255) / 256, nq), 256, 0, s>>>(qrot, P, lut);
}

void launch_row_norms(const float *x, uint32_t rows, uint32_t P, float *out, hipStream_t s) {
    if (rows)
        row_norms_kernel<<<rows < (1u << 20) ? rows : (1u << 20), 64, 0, s>>>(x, rows, P, out);
}

void launch_dist_gemm(const float *q, const float *qnorm, const float *c, const float *cnorm,
                      uint32_t nq, uint32_t nl, uint32_t P, float *dist, hipStream_t s) {
    dim3 grid((nl + kTile - 1) / kTile, (nq + kTile - 1) / kTile);
    const bool vec = P % 4 == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(c) & 15) == 0;
    if (vec) {
        // a slice reads k0 .. k0 + 31 with bounds per 4-float group, so any K % 4 == 0 works
        dim3 g2((nl + kDT - 1) / kDT, (nq + kDT - 1) / kDT);
        dist_gemm_kernel<32><<<g2, 256, 0, s>>>(q, c, dist, nq, nl, P, qnorm, cnorm);
    } else
        gemm_kernel<true, false><<<grid, 256, 0, s>>>(q, c, dist, nq, nl, P, qnorm, cnorm);
}

void launch_split_f16(const float *x, uint32_t rows, uint32_t P, uint16_t *hl, float *scale,
                      hipStream_t s) {
    launch_split_f16_rows(x, rows, P, hl, hl + (size_t)rows * P, scale, s);
}

void launch_split_f16_rows(const float *x, uint32_t rows, uint32_t P, uint16_t *hi, uint16_t *lo, float *scale,
                           hipStream_t s) {
    if (!rows)
        return;
    split_f16_kernel<<<rows < (1u << 20) ? rows : (1u << 20), 64, 0, s>>>(
        x, rows, P, reinterpret_cast<_Float16 *>(hi), reinterpret_cast<_Float16 *>(lo), scale);
}

bool dist_gemm_f16x3_supported(uint32_t K, uint64_t rows_a, uint64_t rows_b) {
    // K % 32: whole MFMA steps (rows then also 16-byte aligned); 32-bit element offsets
    return K % kHK == 0 && rows_a * K < (1ull << 31) && rows_b * K < (1ull << 31);
}

void launch_dist_gemm_f16x3(const uint16_t *qhl, const float *qscale, const float *qnorm,
                            const uint16_t *chl, const float *cscale, const float *cnorm, uint32_t nq,
                            uint32_t nl, uint32_t P, float *dist, hipStream_t s) {
    if (!nq || !nl)
        return;
    const uint32_t nrt = (nq + kHT - 1) / kHT, nct = (nl + kHT - 1) / kHT;
    const uint32_t ncx = (nct + kNumXcd - 1) / kNumXcd, groups = (nrt + 3) / 4;
    const _Float16 *qh = reinterpret_cast<const _Float16 *>(qhl);
    const _Float16 *ch = reinterpret_cast<const _Float16 *>(chl);
    dist_gemm_f16x3_kernel<1><<<kNumXcd * ncx * 4 * groups, 256, 0, s>>>(
        qh, qh + (size_t)nq * P, qscale, ch, ch + (size_t)nl * P, cscale, dist, nq, nl, P, qnorm, cnorm, ncx,
        groups * 4 * kHT, nullptr, nullptr, nullptr, 0);
}

bool fused_probe_supported(uint32_t nl, uint32_t nprobe) {
    // nprobe <= 64: the merge's bound takes the k-th of 64 lane minima (every lane a tile);
    // above, kProbeSlotsWide slots a tile while the tiles hold at most ~4.5 probes each on
    // average (nl / 8 keys per query), and the large-k merge's limits. The candidates fit in
    // the distance matrix they replace.
    if (nprobe < 1 || nl < 64 * kHT || nl > kFusedProbeMaxList)
        return false;
    if (nprobe <= 64)
        return true;
    const uint64_t ntiles = (nl + kHT - 1) / kHT;
    return nprobe <= kMergeBigMaxProbe && (uint64_t)nprobe * 2 * kHT <= 9ull * nl &&
           ntiles * kProbeSlotsWide <= (uint64_t)kMergeBigPer * kMergeBigThreads;
}

uint32_t fused_probe_slots(uint32_t nprobe) { return nprobe <= 64 ? kProbeSlots : kProbeSlotsWide; }

size_t fused_probe_scratch_bytes(uint32_t nq, uint32_t nl, uint32_t nprobe) {
    return (size_t)nq * ((nl + kHT - 1) / kHT) * fused_probe_slots(nprobe) * sizeof(unsigned long long);
}

namespace {
struct FusedGeometry {
    uint32_t nct, ncx, groups;
    const _Float16 *qh, *ch;
    FusedGeometry(const uint16_t *qhl, const uint16_t *chl, uint32_t nq, uint32_t nl)
        : nct((nl + kHT - 1) / kHT), ncx((nct + kNumXcd - 1) / kNumXcd),
          groups(((nq + kHT - 1) / kHT + 3) / 4), qh(reinterpret_cast<const _Float16 *>(qhl)),
          ch(reinterpret_cast<const _Float16 *>(chl)) {}
};
}  // namespace

void launch_fused_probe_gemm(const uint16_t *qhl, const float *qscale, const float *qnorm, const uint16_t *chl,
                             const float *cscale, const float *cnorm, uint32_t nq, uint32_t nl, uint32_t P,
                             uint32_t nprobe, void *scratch, uint32_t *fb, hipStream_t s) {
    if (!nq)
        return;
    // fb: [0] the fallback count, [1 .. nq] the fallback query rows
    launch_fill_u32(fb, 0u, 1, s);
    launch_fused_probe_gemm_rows(qhl, qhl + (size_t)nq * P, qscale, qnorm, chl, cscale, cnorm, 0, nq, nq, nl, P,
                                 nprobe, scratch, s);
}

void launch_fused_probe_gemm_rows(const uint16_t *qhi, const uint16_t *qlo, const float *qscale, const float *qnorm,
                                  const uint16_t *chl, const float *cscale, const float *cnorm, uint32_t r0,
                                  uint32_t rows, uint32_t nq, uint32_t nl, uint32_t P, uint32_t nprobe,
                                  void *scratch, hipStream_t s) {
    if (!rows)
        return;
    // rows [r0, r0 + rows) of the [nq] query operands, as a GEMM of its own whose candidate
    // keys land in those rows of the [nq][nct][slots] candidate array
    const FusedGeometry f(qhi, chl, rows, nl);
    const _Float16 *lo = reinterpret_cast<const _Float16 *>(qlo);
    const uint32_t slots = fused_probe_slots(nprobe);
    auto *cand = static_cast<unsigned long long *>(scratch) + (size_t)r0 * f.nct * slots;
    const dim3 grid(kNumXcd * f.ncx * 4 * f.groups);
    if (slots == kProbeSlots)
        dist_gemm_f16x3_kernel<2, kProbeSlots><<<grid, 256, 0, s>>>(
            f.qh + (size_t)r0 * P, lo + (size_t)r0 * P, qscale + r0, f.ch, f.ch + (size_t)nl * P, cscale, nullptr,
            rows, nl, P, qnorm + r0, cnorm, f.ncx, f.groups * 4 * kHT, nullptr, nullptr, cand, f.nct);
    else
        dist_gemm_f16x3_kernel<2, kProbeSlotsWide><<<grid, 256, 0, s>>>(
            f.qh + (size_t)r0 * P, lo + (size_t)r0 * P, qscale + r0, f.ch, f.ch + (size_t)nl * P, cscale, nullptr,
            rows, nl, P, qnorm + r0, cnorm, f.ncx, f.groups * 4 * kHT, nullptr, nullptr, cand, f.nct);
    (void)nq;
}

void launch_fused_probe_select(const uint16_t *qhl, const float *qscale, const float *qnorm, const uint16_t *chl,
                               const float *cscale, const float *cnorm, uint32_t nq, uint32_t nl, uint32_t P,
                               uint32_t nprobe, void *scratch, uint32_t *fb, int32_t *idx, hipStream_t s) {
    if (!nq)
        return;
    const FusedGeometry f(qhl, chl, nq, nl);
    if (fused_probe_slots(nprobe) == kProbeSlots) {
        static_assert(kFusedProbeMaxList <= 64 * kMergeTiles * kHT, "every tile's keys in a lane's registers");
        probe_merge_kernel<<<(nq + kMergeWaves - 1) / kMergeWaves, 64 * kMergeWaves, 0, s>>>(
            static_cast<const unsigned long long *>(scratch), nq, f.nct, nprobe, idx, fb, fb + 1);
    } else {
        probe_merge_big_kernel<kProbeSlotsWide><<<nq, kMergeBigThreads, 0, s>>>(
            static_cast<const unsigned long long *>(scratch), nq, f.nct, nprobe, idx, fb, fb + 1);
    }
    // fallback: those rows again as a distance matrix (the candidates are no longer needed, so
    // it takes their memory), a grid of up to kFallbackRowTiles row tiles sweeping the *fb rows
    const uint32_t fgroups = min(f.groups, (uint32_t)kFallbackRowTiles / 4);
    float *dist = static_cast<float *>(scratch);
    dist_gemm_f16x3_kernel<3><<<kNumXcd * f.ncx * 4 * fgroups, 256, 0, s>>>(
        f.qh, f.qh + (size_t)nq * P, qscale, f.ch, f.ch + (size_t)nl * P, cscale, dist, nq, nl, P, qnorm, cnorm,
        f.ncx, fgroups * 4 * kHT, fb + 1, fb, nullptr, 0);
    uint32_t kp = 1;
    while (kp < nprobe)
        kp <<= 1;
    select_rows_kernel<<<min(nq, (uint32_t)kFallbackSelectBlocks), kSelThreads, kp * sizeof(unsigned long long), s>>>(
        dist, nl, nprobe, kp, fb + 1, fb, idx);
}

void launch_rotate_f16x3(const uint16_t *xhl, const float *xscale, const uint16_t *rthl,
                         const float *rtscale, uint32_t nq, uint32_t dim, uint32_t P, float *out,
                         hipStream_t s) {
    launch_rotate_f16x3_rows(xhl, xhl + (size_t)nq * dim, xscale, rthl, rtscale, nq, dim, P, out, s);
}

void launch_rotate_f16x3_rows(const uint16_t *xhi, const uint16_t *xlo, const float *xscale, const uint16_t *rthl,
                              const float *rtscale, uint32_t rows, uint32_t dim, uint32_t P, float *out,
                              hipStream_t s) {
    if (!rows)
        return;
    const uint32_t nrt = (rows + kHT - 1) / kHT, nct = (P + kHT - 1) / kHT;
    const uint32_t ncx = (nct + kNumXcd - 1) / kNumXcd, groups = (nrt + 3) / 4;
    const _Float16 *xh = reinterpret_cast<const _Float16 *>(xhi);
    const _Float16 *rh = reinterpret_cast<const _Float16 *>(rthl);
    dist_gemm_f16x3_kernel<0><<<kNumXcd * ncx * 4 * groups, 256, 0, s>>>(
        xh, reinterpret_cast<const _Float16 *>(xlo), xscale, rh, rh + (size_t)P * dim, rtscale, out, rows, P, dim,
        nullptr, nullptr, ncx, groups * 4 * kHT, nullptr, nullptr, nullptr, 0);
}

// ---- big-k select (nprobe > kSelectMaxProbe, up to 65,536): one 1024-thread block per
// query, with the selection in global scratch [k] instead of LDS ----
constexpr int kBigT = 1024;

// exclusive prefix of v over the block (thread order); s_w holds kBigT / 64 words
__device__ __forceinline__ uint32_t big_exclusive_scan(uint32_t v, uint32_t *s_w, uint32_t &total) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o);
        if (lane >= (uint32_t)o)
            x += y;
    }
    if (lane == 63)
        s_w[wave] = x;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kBigT / 64; ++w) {
        before += (uint32_t)w < wave ? s_w[w] : 0u;
        all += s_w[w];
    }
    __syncthreads();
    total = all;
    return x - v + before;
}

// 1. the k-th smallest order key of the row (radix select, four 8-bit passes over the row);
// 2. compaction in cluster-id order of the keys below it and of the first ties (lowest ids)
//    as (key << 32 | id) into a[0, k);
// 3. a stable LSD radix sort of a by key, 4 bits per pass through b (ties keep id order);
// 4. the sorted ids to idx.
__global__ __launch_bounds__(kBigT) void select_big_kernel(const float *__restrict__ dist, uint32_t nl, uint32_t k,
                                                           unsigned long long *__restrict__ scratch,
                                                           int32_t *__restrict__ idx) {
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_w[kBigT / 64];
    __shared__ uint32_t s_sel[2];
    __shared__ uint32_t s_cnt[16 * kBigT];
    const uint32_t t = threadIdx.x, q = blockIdx.x;
    const float *row = dist + (size_t)q * nl;
    unsigned long long *a = scratch + (size_t)q * 2 * k, *b = a + k;
    // 1. radix select
    uint32_t prefix = 0, pmask = 0, need = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (uint32_t i = t; i < 256; i += kBigT)
            s_hist[i] = 0;
        __syncthreads();
        for (uint32_t i = t; i < nl; i += kBigT) {
            const uint32_t key = order_key(row[i]);
            if ((key & pmask) == prefix)
                atomicAdd(&s_hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (t == 0) {
            uint32_t acc = 0, d = 0;
            while (acc + s_hist[d] < need)
                acc += s_hist[d++];
            s_sel[0] = d;
            s_sel[1] = need - acc;
        }
        __syncthreads();
        prefix |= s_sel[0] << shift;
        pmask |= 255u << shift;
        need = s_sel[1];  // keys equal to the k-th that are taken (ties: the lowest ids)
        __syncthreads();
    }
    const uint32_t kth = prefix;
    // 2. ordered compaction: thread t owns ids [t * per, (t + 1) * per)
    const uint32_t per = (nl + kBigT - 1) / kBigT;
    const uint32_t i0 = min(nl, t * per), i1 = min(nl, i0 + per);
    uint32_t nless = 0, neq = 0;
    for (uint32_t i = i0; i < i1; ++i) {
        const uint32_t key = order_key(row[i]);
        nless += key < kth;
        neq += key == kth;
    }
    uint32_t tot_less = 0, tot_eq = 0;
    uint32_t o_less = big_exclusive_scan(nless, s_w, tot_less);
    uint32_t o_eq = big_exclusive_scan(neq, s_w, tot_eq);
    for (uint32_t i = i0; i < i1; ++i) {
        const uint32_t key = order_key(row[i]);
        const unsigned long long v = ((unsigned long long)key << 32) | i;
        if (key < kth)
            a[o_less++] = v;
        else if (key == kth) {
            if (o_eq < need)
                a[tot_less + o_eq] = v;
            ++o_eq;
        }
    }
    __syncthreads();
    // 3. stable LSD radix sort of a[0, k) by key: thread t owns elements [t * kper, ...)
    const uint32_t kper = (k + kBigT - 1) / kBigT;
    const uint32_t e0 = min(k, t * kper), e1 = min(k, e0 + kper);
    unsigned long long *src = a, *dst = b;
    for (int shift = 32; shift < 64; shift += 4) {
        uint32_t c[16];
#pragma unroll
        for (int d = 0; d < 16; ++d)
            c[d] = 0;
        for (uint32_t e = e0; e < e1; ++e) {
            const uint32_t d = (uint32_t)(src[e] >> shift) & 15u;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                c[j] += d == (uint32_t)j;
        }
#pragma unroll
        for (int d = 0; d < 16; ++d)
            s_cnt[d * kBigT + t] = c[d];
        __syncthreads();
        // exclusive scan over s_cnt in (digit, thread) order: thread t sums 16 consecutive entries
        uint32_t part = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            part += s_cnt[t * 16 + j];
        uint32_t total = 0;
        uint32_t run = big_exclusive_scan(part, s_w, total);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t v = s_cnt[t * 16 + j];
            s_cnt[t * 16 + j] = run;
            run += v;
        }
        __syncthreads();
#pragma unroll
        for (int d = 0; d < 16; ++d)
            c[d] = s_cnt[d * kBigT + t];
        for (uint32_t e = e0; e < e1; ++e) {
            const unsigned long long v = src[e];
            const uint32_t d = (uint32_t)(v >> shift) & 15u;
            uint32_t pos = 0;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (d == (uint32_t)j)
                    pos = c[j]++;
            dst[pos] = v;
        }
        __syncthreads();
        unsigned long long *tmp = src;
        src = dst;
        dst = tmp;
    }
    // eight passes: the sorted keys are back in a
    for (uint32_t e = t; e < k; e += kBigT)
        idx[(size_t)q * k + e] = (int32_t)(uint32_t)(a[e] & 0xFFFFFFFFull);
}

void launch_select(const float *dist, uint32_t nq, uint32_t nl, uint32_t nprobe, int32_t *idx,
                   hipStream_t s) {
    if (nprobe > (uint32_t)kSelectMaxProbe) {
        // (launch_select_big, with its scratch, is the caller's path for this size)
        return;
    }
    uint32_t kp = 1;
    while (kp < nprobe)
        kp <<= 1;
    const size_t sel_bytes = kp * sizeof(unsigned long long);
    const size_t lds = sel_bytes + (size_t)nl * 4;
    if (nl > 8192 && nl <= 32u * 512) {
        // 8,192 < nlist <= 16,384: a 512-thread block per query holds the row in registers
        // (read once; 0.41 ms against 0.67 ms for the wave kernel at 10,000 x 16,384)
        select_regs_kernel<32, 512><<<nq, 512, sel_bytes, s>>>(dist, nl, nprobe, kp, idx);
    } else if (nl > 16384 && kp <= 64 && nl % 4 == 0) {
        // 16,384 < nlist: two streaming passes, per-wave candidates (at 10,000 x 65,536 the
        // search step drops from 12.7 to 11.2 ms against the wave kernel's histogram passes)
        select_stream_kernel<<<nq, kSelThreads, sel_bytes, s>>>(dist, nl, nprobe, kp, idx);
    } else if (kp <= kSelWaveMaxK) {
        const uint32_t per = kSelWaveThreads / 64;
        select_wave_kernel<<<(nq + per - 1) / per, kSelWaveThreads, per * sel_bytes, s>>>(dist, nq, nl, nprobe,
                                                                                        kp, idx);
    } else if (nl <= kSelLdsRow && lds <= kSelMaxDynLds) {
        static bool raised = false;  // dynamic LDS above 64 KB must be allowed explicitly
        if (!raised) {
            if (hipFuncSetAttribute(reinterpret_cast<const void *>(&select_kernel<true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSelMaxDynLds) != hipSuccess)
                (void)hipGetLastError();  // leave no sticky error; a launch above 64 KB then reports it
            raised = true;
        }
        select_kernel<true><<<nq, kSelThreads, lds, s>>>(dist, nl, nprobe, kp, idx);
    } else if (nl <= 32u * kSelBigThreads)
        select_regs_kernel<32><<<nq, kSelBigThreads, sel_bytes, s>>>(dist, nl, nprobe, kp, idx);
    else if (nl <= 64u * kSelBigThreads)
        select_regs_kernel<64><<<nq, kSelBigThreads, sel_bytes, s>>>(dist, nl, nprobe, kp, idx);
    else
        select_kernel<false><<<nq, kSelThreads, sel_bytes, s>>>(dist, nl, nprobe, kp, idx);
}

void launch_select_big(const float *dist, uint32_t nq, uint32_t nl, uint32_t nprobe,
                       unsigned long long *scratch, int32_t *idx, hipStream_t s) {
    select_big_kernel<<<nq, kBigT, 0, s>>>(dist, nl, nprobe, scratch, idx);
}

void launch_probe_refine(const float *qrot, const float *cent, const int32_t *idx, uint32_t nq,
                         uint32_t nprobe, uint32_t P, int metric, float *gadd, float *gerr,
                         float err_scale, hipStream_t s) {
    if (nq == 0)
        return;
    probe_refine_kernel<<<std::min(nq, kRefineGrid), 256, 0, s>>>(qrot, cent, idx, nprobe, P, metric, gadd, gerr,
                                                                  err_scale, nq);
}

}  // namespace cora
