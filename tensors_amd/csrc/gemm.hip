// MFMA GEMMs for Matmul forward and backward on gfx950.
//
//   C = epi(alpha * op(A) op(B) + beta * C)      row-major, see tf_hip.h
//
// One kernel template covers NN, NT, TN and TT: the transpose flags pick how
// each operand tile is staged in LDS rather than materialising a transposed
// copy as the reference does (autograd/ops/MatmulBackward.hpp:29-32,
// nn/Linear.cpp:62).  An operand whose reduction index k is contiguous in
// memory ("K-major": A with trans_a == 0, B with trans_b == 1) is staged as
// [rows][k]; one whose row index is contiguous ("MN-major") as [k][rows].
// Global->LDS copies are then straight 16-byte vector copies in both cases,
// and the MFMA fragment reads differ:
//   K-major : each lane reads 16 consecutive k of its row  -> 4 x ds_read_b128
//   MN-major: each lane reads its row at 16 different k; the wave's two
//             accumulators along that dimension take interleaved rows so one
//             ds_read_b64 serves both                      -> 16 x ds_read_b64
// The reduction order inside a 32-deep k block is permuted (lanes 0-31 feed
// k = s, lanes 32-63 feed k = 16 + s to the s-th MFMA) so that the K-major
// reads are contiguous; the sum is the same, the rounding order differs from
// the reference's sequential loop (tensor/Tensor.cpp:356-360) within fp32
// tolerance.
//
// fp32 tile: 128 x BN x 32 per 256-thread workgroup, BN = 128 or 64 (4 waves
// in 2 x 2, each wave 64 x BN/2 = 2 x BN/64 tiles of v_mfma_f32_32x32x2_f32),
// LDS double buffered with one barrier per k block, global loads for block
// k+1 issued before the MFMAs of block k; interior tiles take an unguarded
// 16-byte load path.  bf16: same structure with v_mfma_f32_32x32x16_bf16 and
// a 64-deep k block.  At most ~74 KB of LDS per workgroup, so two workgroups
// share a CU and fill each other's stalls.
//
// Work distribution: the tile index is remapped so that each of the 8 XCDs
// (which receive workgroups round-robin) owns a contiguous, row-grouped block
// of output tiles, keeping its A and B panels in its own L2.  When there are
// too few tiles to fill the GPU and K is long, K is split across
// workgroups; partial tiles go to a workspace and a second kernel reduces
// them in a fixed order (deterministic, no atomics) and applies the epilogue.
#include "common.hpp"

#include <algorithm>

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int BM = 128;
constexpr int kThreads = 256;

struct GemmParams {
    const void* A;
    const void* B;
    void* C;
    const float* bias;
    float* partial;        // split-K workspace [splits][M][N] (nullptr: write C)
    int64_t lda, ldb, ldc;
    int64_t stride_a, stride_b, stride_c;  // batch strides (elements)
    int M, N, K;
    int tiles_m, tiles_n;
    int kb_per_split;      // k blocks per split-K slice
    int reduce_batch;      // >1: C = sum over that many (A_b, B_b) pairs
    float alpha, beta;
    int epi;
    int row_bias;          // bias indexed by row (m) instead of column (n)
    int out_bf16;
    int vec_a, vec_b;      // 16-byte vector loads legal for A / B
    int pair_c;            // 8-byte paired stores legal for C
};

// Remap a linear workgroup id so that the ids one XCD receives (id % 8 == x)
// cover a contiguous range of tiles, then order tiles in groups of GROUP_M
// tile-rows so concurrently running workgroups share A and B panels.
__device__ __forceinline__ void tile_coords(int wg, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    int id = wg;
    if ((total & 7) == 0) id = (wg & 7) * (total >> 3) + (wg >> 3);
    constexpr int GROUP_M = 4;
    const int group_size = GROUP_M * tiles_n;
    const int g = id / group_size;
    const int first_m = g * GROUP_M;
    const int gm = min(tiles_m - first_m, GROUP_M);
    const int in_g = id - g * group_size;
    tm = first_m + in_g % gm;
    tn = in_g / gm;
}

// ---------------------------------------------------------------------------
// Operand staging.  ELEM = float (fp32 path) or uint16_t (bf16 bits).  A
// tile is ROWS rows x BK k.  K-major LDS layout: [ROWS][BK + PADK];
// MN-major: [BK][ROWS + PADM].  The paddings keep the fragment reads free of
// bank conflicts (b128 row reads for K-major; for MN-major the two lane
// halves read k-rows 16 apart, which the padding moves to the other banks).
// ---------------------------------------------------------------------------
template <typename ELEM, int ROWS, int BK, bool KMAJ>
struct Stage {
    static constexpr int VEC = 16 / sizeof(ELEM);            // elements per 16 B
    static constexpr int PADK = (sizeof(ELEM) == 4) ? 4 : 8;
    static constexpr int PADM = (sizeof(ELEM) == 4) ? 2 : 4;
    static constexpr int LD = KMAJ ? (BK + PADK) : (ROWS + PADM);
    static constexpr int LDS_ELEMS = KMAJ ? ROWS * LD : BK * LD;
    static constexpr int LOADS = ROWS * BK / kThreads / VEC;  // 16-byte loads per thread
    static constexpr int TPR = KMAJ ? BK / VEC : ROWS / VEC;  // threads per stored row
    static constexpr int RPP = kThreads / TPR;                // stored rows per pass
    static_assert(LOADS * kThreads * VEC == ROWS * BK, "tile does not divide among threads");

    uint4 reg[LOADS];

    // Global -> registers for the tile whose first row is row0 and first k is
    // k0.  rows: valid row count of the operand; kend: end of this split's k
    // range.  `fast`: the whole tile is in range and 16-byte loads are legal.
    __device__ __forceinline__ void load(const ELEM* __restrict__ p, int64_t ld, int row0, int rows,
                                         int k0, int kend, bool vec_ok) {
        const int t = threadIdx.x;
        const bool fast = vec_ok && row0 + ROWS <= rows && k0 + BK <= kend;
        if (fast) {
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                const int a = t / TPR + RPP * i, b = (t % TPR) * VEC;
                const ELEM* src = KMAJ ? p + (int64_t)(row0 + a) * ld + (k0 + b)
                                       : p + (int64_t)(k0 + a) * ld + (row0 + b);
                reg[i] = *reinterpret_cast<const uint4*>(src);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int a = t / TPR + RPP * i, b = (t % TPR) * VEC;
            const int r = KMAJ ? row0 + a : row0 + b;
            const int k = KMAJ ? k0 + b : k0 + a;
            const bool full = KMAJ ? (r < rows && k + VEC <= kend) : (k < kend && r + VEC <= rows);
            if (vec_ok && full) {
                const ELEM* src = KMAJ ? p + (int64_t)r * ld + k : p + (int64_t)k * ld + r;
                reg[i] = *reinterpret_cast<const uint4*>(src);
            } else {
                ELEM tmp[VEC];
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    const int rr = KMAJ ? r : r + v;
                    const int kk = KMAJ ? k + v : k;
                    const bool ok = rr < rows && kk < kend;
                    tmp[v] = ok ? (KMAJ ? p[(int64_t)rr * ld + kk] : p[(int64_t)kk * ld + rr]) : ELEM(0);
                }
                reg[i] = *reinterpret_cast<uint4*>(tmp);
            }
        }
    }

    // Registers -> LDS (same thread mapping as load()).
    __device__ __forceinline__ void store(ELEM* __restrict__ lds) const {
        const int t = threadIdx.x;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int a = t / TPR + RPP * i, b = (t % TPR) * VEC;
            if (KMAJ) {
                *reinterpret_cast<uint4*>(lds + a * LD + b) = reg[i];
            } else {
                // MN-major rows are 8-byte aligned only (padding): 2 x 8 B.
                uint2* dst = reinterpret_cast<uint2*>(lds + a * LD + b);
                dst[0] = make_uint2(reg[i].x, reg[i].y);
                dst[1] = make_uint2(reg[i].z, reg[i].w);
            }
        }
    }
};

// ---------------------------------------------------------------------------
// Fragment-to-tile mapping.  A wave owns a 64 x WN block of the tile made of
// 2 x NSUB accumulators of 32 x 32 (v_mfma 32x32 layout: lane l, register r
// hold row 8*(r/4) + 4*(l/32) + r%4, column l%32 of the accumulator).  For a
// K-major operand accumulator i covers rows 32i .. 32i+31 of the wave block;
// for an MN-major operand with two accumulators the rows are interleaved
// (accumulator i takes rows 2l + i), so one 8-byte LDS read feeds both.
// ---------------------------------------------------------------------------
template <bool PAIR>
__device__ __forceinline__ int sub_row(int i, int l) { return PAIR ? 2 * l + i : 32 * i + l; }

__device__ __forceinline__ void emit(const GemmParams& p, int64_t off, float acc, float bias_v, bool relu) {
    float v = p.alpha * acc;
    if (p.beta != 0.0f) v += p.beta * reinterpret_cast<const float*>(p.C)[off];
    v += bias_v;
    if (relu) v = fmaxf(v, 0.0f);
    if (p.out_bf16) reinterpret_cast<uint16_t*>(p.C)[off] = tfd::f32_to_bf16(v);
    else reinterpret_cast<float*>(p.C)[off] = v;
}

// Write the wave's accumulators.  m_base/n_base: first row/column of the
// wave block in C.
template <int NSUB, bool A_PAIR, bool B_PAIR>
__device__ __forceinline__ void store_wave(const GemmParams& p, const v16f (&acc)[2][NSUB], int m_base, int n_base,
                                           int64_t batch_off_c, int split) {
    const int lane = threadIdx.x & 63;
    const int l32 = lane & 31, half = lane >> 5;
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    float* part = p.partial ? p.partial + (int64_t)split * p.M * p.N : nullptr;
#pragma unroll
    for (int j = 0; j < NSUB; ++j) {
        if (B_PAIR && j == 1) break;  // paired columns are written together with j == 0
        const int col = n_base + sub_row<B_PAIR>(j, l32);
        const bool c0 = col < p.N, c1 = B_PAIR && col + 1 < p.N;
        if (!c0) continue;
        const bool col_bias = has_bias && !p.row_bias;
        const float cb0 = col_bias ? p.bias[col] : 0.0f;
        const float cb1 = (col_bias && c1) ? p.bias[col + 1] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m_base + sub_row<A_PAIR>(i, 8 * (r >> 2) + 4 * half + (r & 3));
                if (row >= p.M) continue;
                const float rb = (has_bias && p.row_bias) ? p.bias[row] : 0.0f;
                const float b0 = cb0 + rb, b1 = cb1 + rb;
                if (part) {
                    float* dst = part + (int64_t)row * p.N + col;
                    dst[0] = acc[i][j][r];
                    if (B_PAIR && c1) dst[1] = acc[i][1][r];
                    continue;
                }
                const int64_t off = batch_off_c + (int64_t)row * p.ldc + col;
                if (B_PAIR && c1 && p.pair_c && p.beta == 0.0f && !p.out_bf16) {
                    float v0 = p.alpha * acc[i][0][r] + b0, v1 = p.alpha * acc[i][1][r] + b1;
                    if (relu) { v0 = fmaxf(v0, 0.0f); v1 = fmaxf(v1, 0.0f); }
                    *reinterpret_cast<float2*>(reinterpret_cast<float*>(p.C) + off) = make_float2(v0, v1);
                } else {
                    emit(p, off, acc[i][j][r], b0, relu);
                    if (B_PAIR && c1) emit(p, off + 1, acc[i][1][r], b1, relu);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// fp32 kernel: BK = 32, v_mfma_f32_32x32x2_f32.  Lane half h feeds k = 16h + s
// to the s-th MFMA of a k block.
// ---------------------------------------------------------------------------
template <int BN, bool A_KMAJ, bool B_KMAJ>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(GemmParams p) {
    constexpr int BK = 32;
    constexpr int WN = BN / 2;
    constexpr int NSUB = WN / 32;
    constexpr bool A_PAIR = !A_KMAJ;
    constexpr bool B_PAIR = !B_KMAJ && NSUB == 2;
    using SA = Stage<float, BM, BK, A_KMAJ>;
    using SB = Stage<float, BN, BK, B_KMAJ>;
    __shared__ __attribute__((aligned(16))) float lds_a[2][SA::LDS_ELEMS];
    __shared__ __attribute__((aligned(16))) float lds_b[2][SB::LDS_ELEMS];

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int split = blockIdx.y;
    const int batch = blockIdx.z;
    const float* A = reinterpret_cast<const float*>(p.A) + (int64_t)batch * p.stride_a;
    const float* B = reinterpret_cast<const float*>(p.B) + (int64_t)batch * p.stride_b;
    const int m0 = tm * BM, n0 = tn * BN;
    // k blocks of this split: block kb covers batch element kb / kb_per_b
    // (only when reducing over the batch) and k range [(kb % kb_per_b) * BK, ...).
    const int kb_per_b = (p.K + BK - 1) / BK;
    const int kb_total = kb_per_b * p.reduce_batch;
    const int kb_beg = split * p.kb_per_split;
    const int nk = max(0, min(kb_total, kb_beg + p.kb_per_split) - kb_beg);

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l32 = lane & 31;

    v16f acc[2][NSUB];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NSUB; ++j) acc[i][j] = v16f{};

    SA sa;
    SB sb;
    auto load_block = [&](int kb) {
        const int b = kb / kb_per_b, k0 = (kb - b * kb_per_b) * BK;
        sa.load(A + (int64_t)b * p.stride_a, p.lda, m0, p.M, k0, p.K, p.vec_a);
        sb.load(B + (int64_t)b * p.stride_b, p.ldb, n0, p.N, k0, p.K, p.vec_b);
    };
    if (nk > 0) {
        load_block(kb_beg);
        sa.store(lds_a[0]);
        sb.store(lds_b[0]);
    }
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) load_block(kb_beg + kt + 1);
        float fa[2][16], fb[NSUB][16];
        const float* la = lds_a[cur];
        const float* lb = lds_b[cur];
        if (A_KMAJ) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float* src = la + (wm * 64 + sub_row<false>(i, l32)) * SA::LD + 16 * half;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float4 v = *reinterpret_cast<const float4*>(src + 4 * q);
                    fa[i][4 * q + 0] = v.x; fa[i][4 * q + 1] = v.y;
                    fa[i][4 * q + 2] = v.z; fa[i][4 * q + 3] = v.w;
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                float2 v = *reinterpret_cast<const float2*>(la + (16 * half + s) * SA::LD + wm * 64 + 2 * l32);
                fa[0][s] = v.x;
                fa[1][s] = v.y;
            }
        }
        if (B_KMAJ) {
#pragma unroll
            for (int j = 0; j < NSUB; ++j) {
                const float* src = lb + (wn * WN + sub_row<false>(j, l32)) * SB::LD + 16 * half;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float4 v = *reinterpret_cast<const float4*>(src + 4 * q);
                    fb[j][4 * q + 0] = v.x; fb[j][4 * q + 1] = v.y;
                    fb[j][4 * q + 2] = v.z; fb[j][4 * q + 3] = v.w;
                }
            }
        } else if (B_PAIR) {
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                float2 v = *reinterpret_cast<const float2*>(lb + (16 * half + s) * SB::LD + wn * WN + 2 * l32);
                fb[0][s] = v.x;
                fb[NSUB - 1][s] = v.y;
            }
        } else {
#pragma unroll
            for (int s = 0; s < 16; ++s) fb[0][s] = lb[(16 * half + s) * SB::LD + wn * WN + l32];
        }
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < NSUB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
        if (more) {
            sa.store(lds_a[cur ^ 1]);
            sb.store(lds_b[cur ^ 1]);
        }
        __syncthreads();
    }

    store_wave<NSUB, A_PAIR, B_PAIR>(p, acc, m0 + wm * 64, n0 + wn * WN, (int64_t)batch * p.stride_c, split);
}

// ---------------------------------------------------------------------------
// bf16 kernel: BK = 64, v_mfma_f32_32x32x16_bf16 (lane half h supplies the 8
// consecutive k 16s + 8h .. 16s + 8h + 7 to the s-th MFMA of a k block).
// ---------------------------------------------------------------------------
template <int BN, bool A_KMAJ, bool B_KMAJ>
__global__ __launch_bounds__(kThreads) void gemm_bf16_kernel(GemmParams p) {
    constexpr int BK = 64;
    constexpr int WN = BN / 2;
    constexpr int NSUB = WN / 32;
    constexpr bool A_PAIR = !A_KMAJ;
    constexpr bool B_PAIR = !B_KMAJ && NSUB == 2;
    using SA = Stage<uint16_t, BM, BK, A_KMAJ>;
    using SB = Stage<uint16_t, BN, BK, B_KMAJ>;
    __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][SA::LDS_ELEMS];
    __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][SB::LDS_ELEMS];

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int split = blockIdx.y;
    const int batch = blockIdx.z;
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A) + (int64_t)batch * p.stride_a;
    const uint16_t* B = reinterpret_cast<const uint16_t*>(p.B) + (int64_t)batch * p.stride_b;
    const int m0 = tm * BM, n0 = tn * BN;
    // k blocks of this split: block kb covers batch element kb / kb_per_b
    // (only when reducing over the batch) and k range [(kb % kb_per_b) * BK, ...).
    const int kb_per_b = (p.K + BK - 1) / BK;
    const int kb_total = kb_per_b * p.reduce_batch;
    const int kb_beg = split * p.kb_per_split;
    const int nk = max(0, min(kb_total, kb_beg + p.kb_per_split) - kb_beg);

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l32 = lane & 31;

    v16f acc[2][NSUB];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NSUB; ++j) acc[i][j] = v16f{};

    SA sa;
    SB sb;
    auto load_block = [&](int kb) {
        const int b = kb / kb_per_b, k0 = (kb - b * kb_per_b) * BK;
        sa.load(A + (int64_t)b * p.stride_a, p.lda, m0, p.M, k0, p.K, p.vec_a);
        sb.load(B + (int64_t)b * p.stride_b, p.ldb, n0, p.N, k0, p.K, p.vec_b);
    };
    if (nk > 0) {
        load_block(kb_beg);
        sa.store(lds_a[0]);
        sb.store(lds_b[0]);
    }
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) load_block(kb_beg + kt + 1);
        const uint16_t* la = lds_a[cur];
        const uint16_t* lb = lds_b[cur];
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            const int kk = 16 * s + 8 * half;
            v8bf fa[2], fb[NSUB];
            if (A_KMAJ) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    fa[i] = *reinterpret_cast<const v8bf*>(la + (wm * 64 + sub_row<false>(i, l32)) * SA::LD + kk);
            } else {
                uint16_t t0[8], t1[8];
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    uint32_t w = *reinterpret_cast<const uint32_t*>(la + (kk + v) * SA::LD + wm * 64 + 2 * l32);
                    t0[v] = (uint16_t)(w & 0xffffu);
                    t1[v] = (uint16_t)(w >> 16);
                }
                fa[0] = *reinterpret_cast<v8bf*>(t0);
                fa[1] = *reinterpret_cast<v8bf*>(t1);
            }
            if (B_KMAJ) {
#pragma unroll
                for (int j = 0; j < NSUB; ++j)
                    fb[j] = *reinterpret_cast<const v8bf*>(lb + (wn * WN + sub_row<false>(j, l32)) * SB::LD + kk);
            } else if (B_PAIR) {
                uint16_t t0[8], t1[8];
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    uint32_t w = *reinterpret_cast<const uint32_t*>(lb + (kk + v) * SB::LD + wn * WN + 2 * l32);
                    t0[v] = (uint16_t)(w & 0xffffu);
                    t1[v] = (uint16_t)(w >> 16);
                }
                fb[0] = *reinterpret_cast<v8bf*>(t0);
                fb[NSUB - 1] = *reinterpret_cast<v8bf*>(t1);
            } else {
                uint16_t t0[8];
#pragma unroll
                for (int v = 0; v < 8; ++v) t0[v] = lb[(kk + v) * SB::LD + wn * WN + l32];
                fb[0] = *reinterpret_cast<v8bf*>(t0);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < NSUB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            sa.store(lds_a[cur ^ 1]);
            sb.store(lds_b[cur ^ 1]);
        }
        __syncthreads();
    }

    store_wave<NSUB, A_PAIR, B_PAIR>(p, acc, m0 + wm * 64, n0 + wn * WN, (int64_t)batch * p.stride_c, split);
}

// Split-K reduction: C = epi(alpha * sum_s partial[s] + beta * C), summing the
// splits in ascending order (deterministic).
__global__ void splitk_reduce_kernel(GemmParams p, int splits) {
    const int64_t total = (int64_t)p.M * p.N;
    const int64_t plane = total;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    for (; i < total; i += stride) {
        float s = 0.0f;
        for (int k = 0; k < splits; ++k) s += p.partial[k * plane + i];
        const int row = (int)(i / p.N), col = (int)(i - (int64_t)row * p.N);
        const int64_t off = (int64_t)row * p.ldc + col;
        float v = p.alpha * s;
        if (p.beta != 0.0f) v += p.beta * reinterpret_cast<const float*>(p.C)[off];
        if (has_bias) v += p.row_bias ? p.bias[row] : p.bias[col];
        if (relu) v = fmaxf(v, 0.0f);
        if (p.out_bf16) reinterpret_cast<uint16_t*>(p.C)[off] = tfd::f32_to_bf16(v);
        else reinterpret_cast<float*>(p.C)[off] = v;
    }
}

using KernelFn = void (*)(GemmParams);

template <int BN>
KernelFn pick_f32(bool a_kmaj, bool b_kmaj) {
    if (a_kmaj && b_kmaj) return gemm_f32_kernel<BN, true, true>;
    if (a_kmaj && !b_kmaj) return gemm_f32_kernel<BN, true, false>;
    if (!a_kmaj && b_kmaj) return gemm_f32_kernel<BN, false, true>;
    return gemm_f32_kernel<BN, false, false>;
}

template <int BN>
KernelFn pick_bf16(bool a_kmaj, bool b_kmaj) {
    if (a_kmaj && b_kmaj) return gemm_bf16_kernel<BN, true, true>;
    if (a_kmaj && !b_kmaj) return gemm_bf16_kernel<BN, true, false>;
    if (!a_kmaj && b_kmaj) return gemm_bf16_kernel<BN, false, true>;
    return gemm_bf16_kernel<BN, false, false>;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

tf_status gemm_impl(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                    const void* A, int64_t lda, int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b,
                    float beta, void* C, int64_t ldc, int64_t stride_c, int64_t batch, int reduce_batch,
                    int in_dtype, int out_dtype, int epi, const float* bias) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "tf_gemm: negative extent");
    TF_REQUIRE(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31), "tf_gemm: extent exceeds 2^31");
    TF_REQUIRE(stride_a >= 0 && stride_b >= 0 && stride_c >= 0, "tf_gemm: negative batch stride");
    if (M == 0 || N == 0 || batch == 0) return TF_OK;
    TF_REQUIRE(A && B && C, "tf_gemm: null matrix pointer");
    TF_REQUIRE(in_dtype == TF_F32 || in_dtype == TF_BF16, "tf_gemm: in_dtype must be Float32 or BFloat16");
    TF_REQUIRE(out_dtype == TF_F32 || out_dtype == TF_BF16, "tf_gemm: out_dtype must be Float32 or BFloat16");
    TF_REQUIRE(beta == 0.0f || out_dtype == TF_F32, "tf_gemm: beta != 0 needs a Float32 output");
    TF_REQUIRE(epi >= TF_EPI_NONE && epi <= TF_EPI_ROW_BIAS_RELU, "tf_gemm: bad epilogue");
    const bool row_bias = epi == TF_EPI_ROW_BIAS || epi == TF_EPI_ROW_BIAS_RELU;
    TF_REQUIRE(!(epi == TF_EPI_BIAS || epi == TF_EPI_BIAS_RELU || row_bias) || bias != nullptr,
               "tf_gemm: epilogue needs bias");
    // Leading dimensions must cover the stored row length.
    TF_REQUIRE(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N) && ldc >= N, "tf_gemm: leading dimension too small");
    TF_REQUIRE(batch < 65536, "tf_gemm: batch exceeds 65535");
    TF_REQUIRE(!reduce_batch || batch * ((K + 31) / 32) < (1LL << 31), "tf_gemm: reduced K too long");

    const bool a_kmaj = trans_a == 0;  // A[m*lda + k]
    const bool b_kmaj = trans_b != 0;  // B[n*ldb + k]
    const int esz = in_dtype == TF_F32 ? 4 : 2;
    const int vec_elems = 16 / esz;
    const int BK = in_dtype == TF_F32 ? 32 : 64;
    const int64_t grid_batch = reduce_batch ? 1 : batch;

    GemmParams p{};
    p.A = A; p.B = B; p.C = C; p.bias = bias; p.partial = nullptr;
    p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    p.stride_a = stride_a; p.stride_b = stride_b; p.stride_c = reduce_batch ? 0 : stride_c;
    p.M = (int)M; p.N = (int)N; p.K = (int)K;
    // Tile width: 128 x 128 when that gives every CU at least two workgroups
    // (two resident workgroups per CU hide each other's barrier and LDS
    // latency), 128 x 64 otherwise and for narrow outputs.
    const int64_t tiles_m = (M + BM - 1) / BM;
    const int64_t t128 = tiles_m * ((N + 127) / 128) * grid_batch;
    const int BN = (N <= 64 || t128 < 2 * (int64_t)ctx->num_cus) ? 64 : 128;
    p.tiles_m = (int)tiles_m;
    p.tiles_n = (int)((N + BN - 1) / BN);
    p.alpha = alpha; p.beta = beta; p.epi = epi; p.row_bias = row_bias;
    p.out_bf16 = out_dtype == TF_BF16;
    p.reduce_batch = reduce_batch ? (int)batch : 1;
    p.vec_a = aligned16(A) && (lda % vec_elems == 0) && (stride_a % vec_elems == 0);
    p.vec_b = aligned16(B) && (ldb % vec_elems == 0) && (stride_b % vec_elems == 0);
    p.pair_c = (reinterpret_cast<uintptr_t>(C) & 7) == 0 && (ldc % 2 == 0) && (p.stride_c % 2 == 0);

    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    TF_REQUIRE(tiles < (1LL << 31), "tf_gemm: too many tiles");

    // Split the k blocks when the tiles leave most CUs idle and K is long.
    const int64_t kblocks = ((K + BK - 1) / BK) * p.reduce_batch;
    int splits = 1;
    if (grid_batch == 1 && tiles * 2 <= ctx->num_cus && kblocks >= 8) {
        int64_t want = (2 * (int64_t)ctx->num_cus + tiles - 1) / tiles;  // two workgroups per CU
        int64_t max_by_k = kblocks / 4;                                  // >= 4 k blocks per split
        splits = (int)std::max<int64_t>(1, std::min<int64_t>({want, max_by_k, 256}));
    }
    if (kblocks == 0) {
        splits = 1;
        p.kb_per_split = 0;
    } else {
        int64_t per = (kblocks + splits - 1) / splits;
        splits = (int)((kblocks + per - 1) / per);
        p.kb_per_split = (int)per;
    }

    if (splits > 1) {
        size_t need = (size_t)splits * (size_t)M * (size_t)N * sizeof(float);
        tf_status st = tfh::ensure_workspace(ctx, need);
        if (st != TF_OK) return st;
        p.partial = reinterpret_cast<float*>(ctx->ws);
    }

    KernelFn fn = in_dtype == TF_F32 ? (BN == 128 ? pick_f32<128>(a_kmaj, b_kmaj) : pick_f32<64>(a_kmaj, b_kmaj))
                                     : (BN == 128 ? pick_bf16<128>(a_kmaj, b_kmaj) : pick_bf16<64>(a_kmaj, b_kmaj));
    dim3 grid((unsigned)tiles, (unsigned)splits, (unsigned)grid_batch);
    fn<<<grid, kThreads, 0, ctx->stream>>>(p);
    tf_status st = tfh::check_launch("gemm kernel");
    if (st != TF_OK) return st;
    if (splits > 1) {
        splitk_reduce_kernel<<<tfd::grid_for(M * N, 4), 256, 0, ctx->stream>>>(p, splits);
        st = tfh::check_launch("splitk_reduce_kernel");
    }
    return st;
}

}  // namespace

extern "C" {

tf_status tf_gemm(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                  const void* A, int64_t lda, const void* B, int64_t ldb, float beta, void* C, int64_t ldc,
                  int in_dtype, int out_dtype, int epilogue, const float* bias) {
    return gemm_impl(ctx, trans_a, trans_b, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1, 0,
                     in_dtype, out_dtype, epilogue, bias);
}

tf_status tf_gemm_strided_batched(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                                  float alpha, const void* A, int64_t lda, int64_t stride_a, const void* B,
                                  int64_t ldb, int64_t stride_b, float beta, void* C, int64_t ldc,
                                  int64_t stride_c, int64_t batch, int in_dtype, int out_dtype) {
    return gemm_impl(ctx, trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                     stride_c, batch, 0, in_dtype, out_dtype, TF_EPI_NONE, nullptr);
}

tf_status tf_gemm_ex(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                     const void* A, int64_t lda, int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b,
                     float beta, void* C, int64_t ldc, int64_t stride_c, int64_t batch, int reduce_batch,
                     int in_dtype, int out_dtype, int epilogue, const float* bias) {
    return gemm_impl(ctx, trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                     stride_c, batch, reduce_batch, in_dtype, out_dtype, epilogue, bias);
}

}  // extern "C"
