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
#include <type_traits>
#include <utility>

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
// Native 4- and 2-float vectors (HIP's float4 is a struct whose copies lower
// to memcpy, which keeps staging arrays out of registers).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
// Native 16-byte vector (HIP's uint4 is a struct whose copies lower to
// memcpy, which keeps staging arrays out of registers).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128;
constexpr int kThreads = 256;

// Lambdas in the kernels must inline: an out-of-line lambda takes its
// captures (accumulators, staging registers) through memory.
#define TF_LAMBDA_INLINE __attribute__((always_inline))

// Calls f(std::integral_constant<int, I>) for I = 0 .. N-1 (compile-time unroll).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

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
    int vec_c4;            // 4-element vector stores legal for C (16 bytes fp32, 8 bytes bf16)
    uint32_t a_bytes, b_bytes;  // byte extent of one batch element of A / B (buffer loads)
    int int_m, int_n;           // large-tile path: tile rows / columns covered by the direct kernel
    const float* mask_a;        // small fp32 path: A(m, k) taken as A(m, k) * (mask(m, k) > 0), mask laid out as A
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

// Tile of an edge-kernel workgroup.  With an interior grid of int_m x int_n
// tiles (taken by a direct-to-LDS kernel): the tile rows from int_m on, then
// the tile columns from int_n on of the rows above; without one, all tiles.
__device__ __forceinline__ void edge_coords(const GemmParams& p, int& tm, int& tn) {
    if (p.int_m * p.int_n == 0) {
        tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
        return;
    }
    const int id = blockIdx.x;
    const int below = (p.tiles_m - p.int_m) * p.tiles_n;
    if (id < below) {
        tm = p.int_m + id / p.tiles_n;
        tn = id % p.tiles_n;
    } else {
        const int w = p.tiles_n - p.int_n, id2 = id - below;
        tm = id2 / w;
        tn = p.int_n + id2 % w;
    }
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
// wave block in C.  i_only >= 0: only sub-tile row block i_only.
template <int NSUB, bool A_PAIR, bool B_PAIR>
__device__ __forceinline__ void store_wave(const GemmParams& p, const v16f (&acc)[2][NSUB], int m_base, int n_base,
                                           int64_t batch_off_c, int split, int i_only = -1) {
    const int lane = threadIdx.x & 63;
    const int l32 = lane & 31, half = lane >> 5;
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    float* part = p.partial ? p.partial + (int64_t)split * p.M * p.N : nullptr;
    // LOADS: the general form (beta * C, row bias).  Without it no global
    // load sits among the stores: this GPU counts loads and stores in one
    // counter, so a wait for any load also waits for every earlier store.
    auto body = [&](auto LOADS) TF_LAMBDA_INLINE {
        constexpr bool loads = decltype(LOADS)::value;
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
                if (i_only >= 0 && i != i_only) continue;  // the other sub-tile row block is another wave's
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m_base + sub_row<A_PAIR>(i, 8 * (r >> 2) + 4 * half + (r & 3));
                    if (row >= p.M) continue;
                    if (part) {
                        float* dst = part + (int64_t)row * p.N + col;
                        dst[0] = acc[i][j][r];
                        if (B_PAIR && c1) dst[1] = acc[i][1][r];
                        continue;
                    }
                    const int64_t off = batch_off_c + (int64_t)row * p.ldc + col;
                    if constexpr (loads) {
                        const float rb = (has_bias && p.row_bias) ? p.bias[row] : 0.0f;
                        emit(p, off, acc[i][j][r], cb0 + rb, relu);
                        if (B_PAIR && c1) emit(p, off + 1, acc[i][1][r], cb1 + rb, relu);
                    } else {
                        float v0 = p.alpha * acc[i][j][r] + cb0;
                        float v1 = B_PAIR ? p.alpha * acc[i][1][r] + cb1 : 0.0f;
                        if (relu) {
                            v0 = fmaxf(v0, 0.0f);
                            v1 = fmaxf(v1, 0.0f);
                        }
                        if (p.out_bf16) {
                            uint16_t* c = reinterpret_cast<uint16_t*>(p.C) + off;
                            c[0] = tfd::f32_to_bf16(v0);
                            if (B_PAIR && c1) c[1] = tfd::f32_to_bf16(v1);
                        } else if (B_PAIR && c1 && p.pair_c) {
                            *reinterpret_cast<float2*>(reinterpret_cast<float*>(p.C) + off) = make_float2(v0, v1);
                        } else {
                            float* c = reinterpret_cast<float*>(p.C) + off;
                            c[0] = v0;
                            if (B_PAIR && c1) c[1] = v1;
                        }
                    }
                }
            }
        }
    };
    if (p.partial == nullptr && (p.beta != 0.0f || (has_bias && p.row_bias))) body(std::true_type{});
    else body(std::false_type{});
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

// ---------------------------------------------------------------------------
// Large-tile bf16 kernel: 256 x 256 x 64 per 256-thread workgroup, each wave
// a 128 x 128 block (4 x 4 accumulators of 32 x 32, 256 accumulator
// registers).  Per 16-deep k step a wave reads 8 KB of fragments for 16
// MFMAs, half the LDS traffic per flop of a 64 x 64 wave block.
//
// Both operands are kept K-major in LDS ([256 rows][64 k], 128 B per row) so
// every fragment is one ds_read_b128.  The 16-byte chunk c of row r sits at
// chunk position c ^ swz(r); with swz(r) = (r ^ r >> 3) & 7 the 16 lanes of
// a b128 access (16 consecutive rows, one chunk) hit 64 distinct banks.
// MN-major operands are transposed on the way in: each thread loads an
// 8 (k) x 8 (rows) block with eight 16-byte loads and rebuilds eight
// k-contiguous rows in registers (byte permutes).  Threads with mb & 8 write
// their rows in pairwise-swapped order so every 16-lane store group covers
// both row parities, which keeps those stores conflict-free too.
//
// 2 x 32 KB x 2 (double buffer) = 128 KB of LDS: one workgroup per CU.
// ---------------------------------------------------------------------------
constexpr int kBigTile = 256;
constexpr int kBigK = 64;

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

// One 16-byte chunk of bf16 values at p[0 .. 7] with elements i >= n read as
// zero (n <= 0: all zero).
__device__ __forceinline__ u32x4 load_bf16x8_guarded(const uint16_t* __restrict__ p, int n, bool vec_ok) {
    if (vec_ok && n >= 8) return *reinterpret_cast<const u32x4*>(p);
    uint32_t d[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t lo = 2 * w < n ? p[2 * w] : 0u;
        const uint32_t hi = 2 * w + 1 < n ? p[2 * w + 1] : 0u;
        d[w] = lo | (hi << 16);
    }
    return u32x4{d[0], d[1], d[2], d[3]};
}

// Global -> registers -> LDS staging of one 256 x 64 operand tile.  GUARD:
// clip rows to `rows` and k to `kend` (zero fill); without it the caller
// guarantees the whole tile is in range and 16-byte loads are legal.
template <bool KMAJ, bool GUARD>
struct BigStage {
    u32x4 reg[8];  // indexed only through static_for: must stay in registers

    __device__ __forceinline__ void load(const uint16_t* __restrict__ p, int64_t ld, int row0, int rows, int k0,
                                         int kend, bool vec_ok) {
        const int t = threadIdx.x;
        if (KMAJ) {
            // reg[i]: row t/8 + 32i of the tile, k chunk t%8 (8 values).
            const int c = t & 7, r = t >> 3;
            const uint16_t* src = p + (int64_t)(row0 + r) * ld + k0 + 8 * c;
            static_for<8>([&](auto I) TF_LAMBDA_INLINE {
                constexpr int i = decltype(I)::value;
                if (!GUARD) {
                    reg[i] = *reinterpret_cast<const u32x4*>(src + (int64_t)32 * i * ld);
                } else {
                    const bool in = row0 + r + 32 * i < rows;
                    reg[i] = in ? load_bf16x8_guarded(src + (int64_t)32 * i * ld, kend - (k0 + 8 * c), vec_ok)
                                : u32x4{0u, 0u, 0u, 0u};
                }
            });
        } else {
            // Block (kb, mb) = (t/32, t%32): reg[kk] = rows 8mb .. 8mb+7 at k = 8kb + kk.
            const int mb = t & 31, kb = t >> 5;
            const uint16_t* src = p + (int64_t)(k0 + 8 * kb) * ld + row0 + 8 * mb;
            static_for<8>([&](auto KK) TF_LAMBDA_INLINE {
                constexpr int kk = decltype(KK)::value;
                if (!GUARD) {
                    reg[kk] = *reinterpret_cast<const u32x4*>(src + (int64_t)kk * ld);
                } else {
                    const bool in = k0 + 8 * kb + kk < kend;
                    reg[kk] = in ? load_bf16x8_guarded(src + (int64_t)kk * ld, rows - (row0 + 8 * mb), vec_ok)
                                 : u32x4{0u, 0u, 0u, 0u};
                }
            });
        }
    }

    __device__ __forceinline__ void store(u32x4* __restrict__ lds) const {
        const int t = threadIdx.x;
        if (KMAJ) {
            const int c = t & 7, r = t >> 3;
            static_for<8>([&](auto I) TF_LAMBDA_INLINE {
                constexpr int i = decltype(I)::value;
                const int row = r + 32 * i;
                lds[row * 8 + (c ^ swz(row))] = reg[i];
            });
        } else {
            const int mb = t & 31, kb = t >> 5;
            const int flip = (mb >> 3) & 1;
            const uint32_t keep = flip ? 0u : ~0u;  // bit blend, not a runtime index
            // Row 8mb + m as 4 bf16 pairs: pair j = (k 2j, k 2j+1) = element m of reg[2j], reg[2j+1].
            auto row_words = [&](auto M) TF_LAMBDA_INLINE {
                constexpr int m = decltype(M)::value;
                uint32_t d[4];
                static_for<4>([&](auto J) TF_LAMBDA_INLINE {
                    constexpr int j = decltype(J)::value;
                    const uint32_t lo = reg[2 * j][m >> 1];
                    const uint32_t hi = reg[2 * j + 1][m >> 1];
                    d[j] = (m & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
                });
                return u32x4{d[0], d[1], d[2], d[3]};
            };
            static_for<8>([&](auto J) TF_LAMBDA_INLINE {
                constexpr int j = decltype(J)::value;
                const u32x4 x = row_words(std::integral_constant<int, j>{});
                const u32x4 y = row_words(std::integral_constant<int, j ^ 1>{});
                const u32x4 v = (x & keep) | (y & ~keep);
                const int row = 8 * mb + (j ^ flip);
                lds[row * 8 + (kb ^ swz(row))] = v;
            });
        }
    }
};

// Fragments of k step s (0..3) of an LDS block: lane half h feeds
// k = 16s + 8h .. +7, i.e. chunk 2s + h of its row.  a_row/b_row: u32x4
// offsets of the lane's four A and B rows; a_sw/b_sw: their swizzles.
struct BigFrags {
    v8bf a[4], b[4];
};

__device__ __forceinline__ void big_read(const u32x4* __restrict__ la, const u32x4* __restrict__ lb, int s,
                                         const int (&a_row)[4], const int (&a_sw)[4], const int (&b_row)[4],
                                         const int (&b_sw)[4], int half, BigFrags& f) {
    const int c = 2 * s + half;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f.a[i] = __builtin_bit_cast(v8bf, la[a_row[i] + (c ^ a_sw[i])]);
        f.b[i] = __builtin_bit_cast(v8bf, lb[b_row[i] + (c ^ b_sw[i])]);
    }
}

__device__ __forceinline__ void big_mfma(const BigFrags& f, v16f (&acc)[4][4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// MFMAs BEGIN .. END-1 of the 16 of one k step (index 4i + j).
template <int BEGIN, int END>
__device__ __forceinline__ void big_mfma_part(const BigFrags& f, v16f (&acc)[4][4]) {
#pragma unroll
    for (int x = BEGIN; x < END; ++x)
        acc[x >> 2][x & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[x >> 2], f.b[x & 3], acc[x >> 2][x & 3], 0, 0, 0);
}

// Eight-wave form (a 128 x 64 block per wave, two waves per SIMD): four A and
// two B fragments per k step, 8 MFMAs (index 2i + j).
struct BigFrags8 {
    v8bf a[4], b[2];
};
__device__ __forceinline__ void big_mfma8(const BigFrags8& f, v16f (&acc)[4][2]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}
template <int BEGIN, int END>
__device__ __forceinline__ void big_mfma8_part(const BigFrags8& f, v16f (&acc)[4][2]) {
#pragma unroll
    for (int x = BEGIN; x < END; ++x)
        acc[x >> 1][x & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[x >> 1], f.b[x & 1], acc[x >> 1][x & 1], 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Interior tiles (gemm_bf16_dl_kernel): operands go global -> LDS directly
// with buffer_load_dwordx4 ... lds (no registers, no LDS write
// instructions), 32-deep k blocks in 5 LDS buffers of 2 x 16 KB, so four
// blocks (128 KB) are in flight while one is computed.  Loads are issued
// about seven 16-deep k steps ahead of use, which covers the L2/HBM round
// trip at full MFMA rate.
//
// A wave's load instruction fills 1 KB of LDS, lane l bytes 16l .. 16l+15,
// so the swizzle is applied to the global addresses:
//   K-major operand, LDS [256 rows][32 k] (64 B rows, 4 chunks): 1 KB = 16
//     rows; lane l loads row l/4, logical chunk (l%4) ^ swz32(row) with
//     swz32(row) = (row >> 2) & 3, which spreads the 16 rows of one b128
//     fragment read over all 64 banks.  Fragments: ds_read_b128.
//   MN-major operand, LDS [32 k][256 rows] (512 B per k row): 1 KB = 2 k
//     rows; lane l loads k row l/32, logical chunk (l%32) ^ 4(k%4).
//     Fragments: ds_read_b64_tr_b16, which hands lane i (of each 16-lane
//     group) element i%4 of the 8-byte rows addressed by lanes i/4 + 4j,
//     j = 0..3: with lane a addressing [k = kb + a/4][m = mb + 4(a%4)], lane
//     i receives A[mb + i][kb + j], the MFMA operand layout.  The chunk
//     rotation by 4(k%4) spreads the four k rows of one read over all banks.
// ---------------------------------------------------------------------------
constexpr int kDlK = 32;                                  // k per LDS block
constexpr int kDlBufs = 5;                                // LDS blocks
constexpr int kDlVec = kBigTile * kDlK * 2 / 16;          // u32x4 per operand block (16 KB)
constexpr int kDlLoads = kBigTile * kDlK * 2 / 1024 / 4;  // 1 KB loads per wave per operand block
constexpr int kDl8Loads = kDlLoads / 2;                    // the same with eight waves

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(lds_void_ptr)const_cast<void*>(p);
}
// LDS byte offset of this wave's 1 KB pieces of a direct-load block (wave w
// fills pieces loads*w ..), as a scalar.
template <int LOADS>
__device__ __forceinline__ uint32_t dl_wave_offset() {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6) * LOADS * 1024);
}

__device__ __forceinline__ int swz32(int row) { return (row >> 2) & 3; }

using tfd::waitcnt_vm;
using tfd::waitcnt_vm_lds;

// Workgroup barrier for the direct-to-LDS pipeline: waits for this wave's
// loads except the newest `outstanding` and for all of its LDS reads, then
// s_barrier.  __syncthreads() would add a release fence, which must wait for
// every in-flight LDS load (vmcnt(0)) and so would drain the pipeline.  The
// "memory" clobber keeps the compiler from moving memory accesses across.
template <int OUTSTANDING>
__device__ __forceinline__ void dl_barrier() {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lds(OUTSTANDING));
    asm volatile("s_barrier" ::: "memory");
}

// Byte offsets (from the operand's base) of this lane's LOADS direct loads
// of a tile at row0 = k0 = 0; the tile position is added as a uniform
// offset.  Wave w fills 1 KB blocks LOADS*w .. of the LDS block (LOADS = 4
// with four waves, 2 with eight).
template <bool KMAJ, int LOADS = kDlLoads>
__device__ __forceinline__ void dl_offsets(int64_t ld, uint32_t (&voff)[LOADS]) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int blk = w * LOADS + i;
        if (KMAJ) {
            const int row = blk * 16 + (l >> 2);
            voff[i] = 2u * ((uint32_t)row * (uint32_t)ld + 8u * (uint32_t)((l & 3) ^ swz32(row)));
        } else {
            const int k = blk * 2 + (l >> 5);
            voff[i] = 2u * ((uint32_t)k * (uint32_t)ld + 8u * (uint32_t)((l & 31) ^ (4 * (k & 3))));
        }
    }
}

// First k (within the 32-deep block) of each of this lane's LOADS direct
// loads, in the layout of dl_offsets: a K-major 16-byte load holds k .. k+7
// of one row, an MN-major one holds row k.  With K % 8 == 0 a load is
// wholly inside or wholly past K.
template <bool KMAJ, int LOADS = kDlLoads>
__device__ __forceinline__ void dl_klane(int (&kl)[LOADS]) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int blk = w * LOADS + i;
        kl[i] = KMAJ ? 8 * ((l & 3) ^ swz32(blk * 16 + (l >> 2))) : blk * 2 + (l >> 5);
    }
}

// Lane offset of a load past K: above any descriptor extent (< 2^31), so the
// buffer range check returns zeros (the lane offset alone is out of range).
constexpr uint32_t kDlOob = 0x80000000u;

// Buffer resource descriptor for raw 16-byte loads from `base` (gfx9-family
// word 3: raw dword access; reads beyond `bytes` return zero).  The range
// check covers the lane offset plus the scalar offset: measured on gfx950,
// a load at scalar offset 2048, lane offset 0 of a 1024-byte descriptor
// returns zeros.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 dl_rsrc(uint64_t a, uint32_t bytes) {
    return i32x4{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), (int)bytes, 0x00020000};
}
__device__ __forceinline__ i32x4 dl_rsrc(const void* base, uint32_t bytes) {
    return dl_rsrc(reinterpret_cast<uint64_t>(base), bytes);
}

// The k blocks a direct kernel loads, in order: kb_beg, kb_beg + 1, ... up
// to the split's last block, then that block again (the clamped loads past
// the end).  Block kb lies in batch element kb / kpb (a batch reduction) at
// k block kb % kpb.  The walk keeps that position and the element's operand
// addresses in scalar registers and advances them with selects, so issuing a
// block costs a few scalar instructions.  Computing them per block (a
// division and 64-bit batch offsets, ~50 scalar instructions next to the
// barrier, where the MFMA pipe waits for them) cost 3-4 % on the large bf16
// GEMMs and 1.5-3 % on the fp32 ones.
struct KWalk {
    uint64_t a_base, b_base;      // byte addresses of the current element's A and B
    uint64_t a_step, b_step;      // bytes between batch elements
    int kin, kpb, left;           // k block in the element; blocks per element; blocks after this one
    __device__ __forceinline__ void init(const void* A, const void* B, int64_t a_stride_bytes, int64_t b_stride_bytes,
                                         int kb_beg, int nk, int kpb_) {
        kpb = kpb_;
        const int b = kb_beg / kpb_;
        kin = kb_beg - b * kpb_;
        a_step = (uint64_t)a_stride_bytes;
        b_step = (uint64_t)b_stride_bytes;
        a_base = reinterpret_cast<uint64_t>(A) + (uint64_t)b * a_step;
        b_base = reinterpret_cast<uint64_t>(B) + (uint64_t)b * b_step;
        left = nk - 1;
    }
    __device__ __forceinline__ void advance() {
        const int adv = left > 0 ? 1 : 0;
        left -= adv;
        const int kn = kin + adv;
        const bool wrap = kn == kpb;
        kin = wrap ? 0 : kn;
        a_base = wrap ? a_base + a_step : a_base;
        b_base = wrap ? b_base + b_step : b_base;
    }
};

// Issue this wave's direct loads of one operand block:
// buffer_load_dwordx4 ... lds, M0 = the 1 KB LDS destination.  Written as
// inline assembly on purpose: the compiler's wait-count tracking of LDS
// loads loses track of which buffer each one writes (at the loop header) and
// then makes fragment reads wait for every load in flight, draining the
// pipeline.  The kernel waits for these loads itself (dl_barrier, and a
// final vmcnt(0)), and nothing else in it uses M0.
// `lds_wave`: LDS byte address of this wave's first 1 KB of the block (a
// scalar computed once per kernel: deriving it per load from the generic
// pointer cost a readfirstlane and a null-check select per load).
template <int LOADS = kDlLoads>
__device__ __forceinline__ void dl_issue(i32x4 rsrc, uint32_t tile_off, const uint32_t (&voff)[LOADS],
                                         uint32_t lds_wave) {
    static_for<LOADS>([&](auto I) TF_LAMBDA_INLINE {
        constexpr int i = decltype(I)::value;
        const uint32_t dst = lds_wave + i * 1024u;
        const uint32_t v = voff[i], so = tile_off;  // asm operands must be locals of the lambda
        const i32x4 r = rsrc;
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                     :
                     : "s"(dst), "v"(v), "s"(r), "s"(so)
                     : "memory", "m0");
    });
}

// Per-lane fragment offsets of one operand (NSUB sub-tiles of 32 rows from
// row wbase).  K-major: u32x4 index of the row and its swizzle.  MN-major:
// bf16 element offset of the lane's first transposed read.
template <bool KMAJ, int NSUB = 4>
struct DlOperand {
    int off[NSUB], sw[NSUB];
    __device__ __forceinline__ void init(int wbase) {
        const int l = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < NSUB; ++i) {
            if (KMAJ) {
                const int r = wbase + 32 * i + (l & 31);
                off[i] = r * (kDlK / 8);
                sw[i] = swz32(r);
            } else {
                const int g = l >> 4, a = l & 15, q = a & 3, j = a >> 2;
                const int m = wbase + 32 * i + 16 * (g & 1) + 4 * q;
                off[i] = (8 * (g >> 1) + j) * kBigTile + (((m >> 3) ^ (4 * j)) * 8) + (m & 7);
                sw[i] = 0;
            }
        }
    }
    // Fragment of sub-tile i at k step s (lane half h: k = 16s + 8h .. +7).
    __device__ __forceinline__ v8bf frag(const u32x4* __restrict__ lds, int i, int s, int half) const {
        if (KMAJ) return __builtin_bit_cast(v8bf, lds[off[i] + ((2 * s + half) ^ sw[i])]);
        const short* base = reinterpret_cast<const short*>(lds) + off[i] + 16 * s * kBigTile;
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)base);
        const v4s hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(base + 4 * kBigTile));
        return __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
};

// Writes a 256 x 256 accumulator tile (bounds-checked when GUARD).
// Epilogue of the 256 x 256 kernels, staged through LDS: each wave writes
// its raw accumulators, 64 rows x 128 columns at a time, into its own 32 KB
// of LDS, then copies them out by whole rows (a lane takes 4 consecutive
// columns, 32 lanes a row), applying alpha, beta * C, bias and ReLU per
// 4-column vector, so C is written with 16-byte (fp32) or 8-byte (bf16)
// stores of contiguous rows.  The copy loop is a run-time loop, so its body
// (every output variant) exists twice in the code rather than once per row
// group: writing the accumulators element by element from fully unrolled
// code instead made the epilogue tens of kilobytes of straight-line code and
// slower than the k loop of a 1000-deep GEMM.  Lane l, register r of
// acc[i][j] is row 32i + 8(r/4) + 4(l/32) + r%4, column 32j + l%32 of the
// wave block; static_for keeps every accumulator index a compile-time
// constant (a runtime index would move the accumulators to scratch).  The
// caller has synchronised the workgroup: `stage` (8192 floats) may alias
// buffers the main loop used.
template <int WCOLS = 128>
__device__ __forceinline__ void big_epilogue(const GemmParams& p, v16f (&acc)[4][WCOLS / 32], int m0, int n0,
                                             int split, int batch, float* __restrict__ stage) {
    constexpr int WN = 256 / WCOLS;    // waves along a tile row
    constexpr int LPR = WCOLS / 4;     // lanes per staged row
    constexpr int RPP = 64 / LPR;      // staged rows per pass
    constexpr int PASSES = 64 / RPP;   // passes per 64 staged rows
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int half = lane >> 5, l32 = lane & 31;   // accumulator layout
    const int rsub = lane / LPR;                   // copy layout: row within a pass
    const int lc = 4 * (lane % LPR);               // this lane's 4 columns of a staged row
    const int col = n0 + wn * WCOLS + lc;
    float* part = p.partial ? p.partial + (int64_t)split * p.M * p.N : nullptr;
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    const float* row_bias = has_bias && p.row_bias ? p.bias : nullptr;
    const bool vec = (part ? (p.N % 4 == 0) : p.vec_c4 != 0) && col + 4 <= p.N;
    float cb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) cb[e] = (has_bias && !p.row_bias && col + e < p.N) ? p.bias[col + e] : 0.0f;
    const float alpha = p.alpha, beta = p.beta;
    const int64_t ldc = p.ldc, boff = (int64_t)batch * p.stride_c;

    // One staged vector: columns col .. col+3 of `row`.  The output form is
    // fixed per loop (template flags) so the copy loop carries no branches on
    // it.  PART: split-K partial (fp32, leading dimension N).  LOADS: the
    // general form (beta * C, row bias); without it the loop holds no global
    // load: this GPU counts loads and stores in one counter, so any load in
    // the loop makes the compiler wait for every store issued before it and
    // serialises the loop on store latency.
    auto out4 = [&](int row, f32x4 v, auto PART, auto BF16, auto LOADS) TF_LAMBDA_INLINE {
        constexpr bool is_part = decltype(PART)::value, bf16 = decltype(BF16)::value;
        constexpr bool loads = decltype(LOADS)::value;
        if constexpr (is_part) {
            float* dst = part + (int64_t)row * p.N + col;
            if (vec) {
                *reinterpret_cast<f32x4*>(dst) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < p.N) dst[e] = v[e];
            }
            return;
        }
        float rb = 0.0f;
        if constexpr (loads) rb = row_bias ? row_bias[row] : 0.0f;
        const int64_t off = boff + (int64_t)row * ldc + col;
        f32x4 old = {0.f, 0.f, 0.f, 0.f};
        if constexpr (loads) {
            if (beta != 0.0f) {
                const float* c = reinterpret_cast<const float*>(p.C) + off;
                if (vec) {
                    old = *reinterpret_cast<const f32x4*>(c);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) old[e] = col + e < p.N ? c[e] : 0.0f;
                }
            }
        }
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float t = alpha * v[e];
            if (loads) t += beta * old[e];
            t += cb[e] + rb;
            o[e] = relu ? fmaxf(t, 0.0f) : t;
        }
        if constexpr (bf16) {
            uint16_t* c = reinterpret_cast<uint16_t*>(p.C) + off;
            if (vec) {
                *reinterpret_cast<uint2*>(c) = make_uint2(tfd::bf16x2_rne(o[0], o[1]), tfd::bf16x2_rne(o[2], o[3]));
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < p.N) c[e] = tfd::f32_to_bf16(o[e]);
            }
        } else {
            float* c = reinterpret_cast<float*>(p.C) + off;
            if (vec) {
                *reinterpret_cast<f32x4*>(c) = o;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < p.N) c[e] = o[e];
            }
        }
    };
    const bool general = !part && (beta != 0.0f || row_bias != nullptr);
    using T_ = std::true_type;
    using F_ = std::false_type;
    static_for<2>([&](auto RND) TF_LAMBDA_INLINE {
        constexpr int rnd = decltype(RND)::value;
        // Sub-tile row blocks 2rnd, 2rnd + 1 -> staged rows 0 .. 63.
        static_for<2>([&](auto II) TF_LAMBDA_INLINE {
            constexpr int ii = decltype(II)::value;
            static_for<WCOLS / 32>([&](auto J) TF_LAMBDA_INLINE {
                constexpr int j = decltype(J)::value;
                static_for<16>([&](auto R) TF_LAMBDA_INLINE {
                    constexpr int r = decltype(R)::value;
                    const int lrow = 32 * ii + 8 * (r >> 2) + 4 * half + (r & 3);
                    stage[lrow * WCOLS + 32 * j + l32] = acc[2 * rnd + ii][j][r];
                });
            });
        });
        const int row0 = m0 + wm * 128 + 64 * rnd + rsub;
        // The LDS read of pass + 1 is issued before pass is written out, so
        // its latency overlaps the conversion and store.
        const float* src = stage + rsub * WCOLS + lc;
        auto copy_out = [&](auto PART, auto BF16, auto LOADS) TF_LAMBDA_INLINE {
            f32x4 next = *reinterpret_cast<const f32x4*>(src);
#pragma unroll 2
            for (int pass = 0; pass < PASSES; ++pass) {
                const f32x4 v = next;
                next = *reinterpret_cast<const f32x4*>(src + min(pass + 1, PASSES - 1) * RPP * WCOLS);
                const int row = row0 + RPP * pass;
                if (row < p.M && col < p.N) out4(row, v, PART, BF16, LOADS);
            }
        };
        // Interior blocks (the wave's 64 x 128 staged block inside C, every
        // 4-column vector aligned) without beta * C or a row bias: no bounds
        // checks, a pointer advanced by two rows per pass, and the transform
        // fixed at compile time (XF 0: copy, 1: alpha * v + bias, 2: the same
        // then ReLU).  OUT 0: split-K partial, 1: bf16 C, 2: fp32 C.  The
        // generic loop above spent most of its time on per-pass address
        // arithmetic, bounds and form checks, and software bf16 rounding.
        auto copy_fast = [&](auto OUT, auto XF) TF_LAMBDA_INLINE {
            constexpr int out = decltype(OUT)::value, xf = decltype(XF)::value;
            using Dst = std::conditional_t<out == 1, uint16_t, float>;
            const int64_t ld = out == 0 ? (int64_t)p.N : ldc;
            Dst* dst = out == 0 ? reinterpret_cast<Dst*>(part) + (int64_t)row0 * ld + col
                                : reinterpret_cast<Dst*>(p.C) + boff + (int64_t)row0 * ld + col;
            f32x4 next = *reinterpret_cast<const f32x4*>(src);
#pragma unroll 2
            for (int pass = 0; pass < PASSES; ++pass) {
                f32x4 o = next;
                next = *reinterpret_cast<const f32x4*>(src + min(pass + 1, PASSES - 1) * RPP * WCOLS);
                if constexpr (xf != 0) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float t = alpha * o[e] + cb[e];
                        o[e] = xf == 2 ? fmaxf(t, 0.0f) : t;
                    }
                }
                if constexpr (out == 1)
                    *reinterpret_cast<uint2*>(dst) = make_uint2(tfd::bf16x2_rne(o[0], o[1]), tfd::bf16x2_rne(o[2], o[3]));
                else
                    *reinterpret_cast<f32x4*>(dst) = o;
                dst += RPP * ld;
            }
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        const bool interior = !general && (part ? p.N % 4 == 0 : p.vec_c4 != 0) &&
                              m0 + wm * 128 + 64 * rnd + 64 <= p.M && n0 + wn * WCOLS + WCOLS <= p.N;
        const bool plain = alpha == 1.0f && !has_bias && !relu;
        if (interior) {
            if (part) copy_fast(I0{}, I0{});
            else if (p.out_bf16) {
                if (plain) copy_fast(I1{}, I0{});
                else if (relu) copy_fast(I1{}, I2{});
                else copy_fast(I1{}, I1{});
            } else {
                if (plain) copy_fast(I2{}, I0{});
                else if (relu) copy_fast(I2{}, I2{});
                else copy_fast(I2{}, I1{});
            }
        } else if (part) copy_out(T_{}, F_{}, F_{});
        else if (general && p.out_bf16) copy_out(F_{}, T_{}, T_{});  // row bias (beta != 0 needs an fp32 C)
        else if (general) copy_out(F_{}, F_{}, T_{});
        else if (p.out_bf16) copy_out(F_{}, T_{}, F_{});
        else copy_out(F_{}, F_{}, F_{});
    });
}

// One 256 x 256 tile with register-staged, bounds-checked 64-deep blocks.
template <bool A_KMAJ, bool B_KMAJ>
__device__ __forceinline__ void big_tile_guarded(const GemmParams& p, int m0, int n0, int split, int batch,
                                                 int kb_beg, int nk, u32x4* a0, u32x4* a1, u32x4* b0, u32x4* b1) {
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A) + (int64_t)batch * p.stride_a;
    const uint16_t* B = reinterpret_cast<const uint16_t*>(p.B) + (int64_t)batch * p.stride_b;
    const int kb_per_b = (p.K + kBigK - 1) / kBigK;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l32 = lane & 31;

    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};

    int a_row[4], a_sw[4], b_row[4], b_sw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ra = wm * 128 + 32 * i + l32, rb = wn * 128 + 32 * i + l32;
        a_row[i] = ra * 8; a_sw[i] = swz(ra);
        b_row[i] = rb * 8; b_sw[i] = swz(rb);
    }

    // Software pipeline over k blocks (LDS buffer kt & 1 holds block kt):
    //   step 0: MFMAs of k step 0 | fragment reads for step 1
    //   step 1: MFMAs of step 1   | reads for step 2
    //   step 2: MFMAs of step 2   | reads for step 3; LDS writes of block
    //                               kt+1 (staged in registers) to the other buffer
    //   barrier                   (block kt+1 complete; block kt-1 no longer read)
    //   step 3: MFMAs of step 3   | global loads of block kt+2 into the staging
    //                               registers; reads of block kt+1's step 0
    // Global loads get three k steps to land; the MFMA pipe is fed across the
    // barrier.  sched_group_barrier pins the interleaving (the default
    // scheduler clusters the memory operations and exposes their latency).
    if (nk > 0) {
        u32x4* lds_a[2] = {a0, a1};
        u32x4* lds_b[2] = {b0, b1};
        BigStage<A_KMAJ, true> sa;
        BigStage<B_KMAJ, true> sb;
        BigFrags f[2];
        auto load_block = [&](int kb) TF_LAMBDA_INLINE {
            const int b = kb / kb_per_b, k0 = (kb - b * kb_per_b) * kBigK;
            sa.load(A + (int64_t)b * p.stride_a, p.lda, m0, p.M, k0, p.K, p.vec_a);
            sb.load(B + (int64_t)b * p.stride_b, p.ldb, n0, p.N, k0, p.K, p.vec_b);
        };
        auto read = [&](int buf, int s, BigFrags& dst) TF_LAMBDA_INLINE {
            big_read(lds_a[buf], lds_b[buf], s, a_row, a_sw, b_row, b_sw, half, dst);
        };
        // One k block.  STORE: block kt+1 is staged and goes to LDS in step 2.
        // LOAD: block kt+2 exists and is loaded in step 3.
        auto block = [&](int kt, auto STORE, auto LOAD) TF_LAMBDA_INLINE {
            constexpr bool store = decltype(STORE)::value, load = decltype(LOAD)::value;
            const int cur = kt & 1;
            static_for<3>([&](auto S) TF_LAMBDA_INLINE {
                constexpr int s = decltype(S)::value;
                read(cur, s + 1, f[(s + 1) & 1]);
                big_mfma(f[s & 1], acc);
                if constexpr (s == 2 && store) {
                    sa.store(lds_a[cur ^ 1]);
                    sb.store(lds_b[cur ^ 1]);
                    static_for<8>([&](auto) TF_LAMBDA_INLINE {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);  // DS write
                    });
                } else {
                    static_for<8>([&](auto) TF_LAMBDA_INLINE {
                        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                    });
                }
                __builtin_amdgcn_sched_barrier(0);
            });
            if constexpr (store) __syncthreads();
            if constexpr (load) load_block(kb_beg + kt + 2);
            if constexpr (store) read(cur ^ 1, 0, f[0]);
            big_mfma(f[1], acc);
            if constexpr (load && store) {
                static_for<8>([&](auto) TF_LAMBDA_INLINE {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // VMEM read
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                });
            } else if constexpr (store) {
                static_for<8>([&](auto) TF_LAMBDA_INLINE {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                });
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        using T = std::true_type;
        using F = std::false_type;
        load_block(kb_beg);
        sa.store(lds_a[0]);
        sb.store(lds_b[0]);
        if (nk > 1) load_block(kb_beg + 1);
        __syncthreads();
        read(0, 0, f[0]);
        int kt = 0;
        for (; kt + 2 < nk; ++kt) block(kt, T{}, T{});
        if (kt + 1 < nk) block(kt++, T{}, F{});
        block(kt, F{}, F{});
    }

    __syncthreads();  // the epilogue stages through the operand buffers (one 32 KB buffer per wave)
    big_epilogue(p, acc, m0, n0, split, batch,
                 reinterpret_cast<float*>(wave == 0 ? a0 : wave == 1 ? a1 : wave == 2 ? b0 : b1));
}

// Interior-tile kernel.  Per 32-deep block t (LDS buffer t % 5):
//   step 0: MFMAs of k step 0 | fragment reads of step 1
//   wait for block t+1's loads (vmcnt), barrier: block t+1 is visible and
//     every wave holds all of block t's fragments
//   step 1: MFMAs of step 1 | loads of block t+5 into buffer t % 5 |
//     reads of block t+1's step 0
// The five LDS buffers are separate objects and every access names its
// buffer at compile time (block<B>), so the compiler can see that a load
// into one buffer does not alias fragment reads from another.
template <bool A_KMAJ, bool B_KMAJ>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_dl_kernel(GemmParams p) {
    // One array per buffer (A block, then B block): the compiler tracks the
    // targets of in-flight LDS loads per LDS object and only for a few
    // objects; with more, every fragment read waits for all loads.
    __shared__ u32x4 s0[2 * kDlVec], s1[2 * kDlVec], s2[2 * kDlVec], s3[2 * kDlVec], s4[2 * kDlVec];

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int split = blockIdx.y;
    const int batch = blockIdx.z;
    const int m0 = tm * kBigTile, n0 = tn * kBigTile;
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A) + (int64_t)batch * p.stride_a;
    const uint16_t* B = reinterpret_cast<const uint16_t*>(p.B) + (int64_t)batch * p.stride_b;
    // Splits are counted in 64-deep blocks (K % 64 == 0 here): two of ours each.
    const int kb64_total = (p.K / 64) * p.reduce_batch;
    const int kb64_beg = split * p.kb_per_split;
    const int nk = 2 * max(0, min(kb64_total, kb64_beg + p.kb_per_split) - kb64_beg);
    const int kb_beg = 2 * kb64_beg;
    const int kpb = p.K / kDlK;  // 32-deep blocks per batch element

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int half = lane >> 5;
    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};

    if (nk > 0) {
        DlOperand<A_KMAJ> oa;
        DlOperand<B_KMAJ> ob;
        oa.init((wave >> 1) * 128);
        ob.init((wave & 1) * 128);
        uint32_t voff_a[kDlLoads], voff_b[kDlLoads];
        dl_offsets<A_KMAJ>(p.lda, voff_a);
        dl_offsets<B_KMAJ>(p.ldb, voff_b);
        BigFrags f[2];
        auto buf_a = [&](auto Bc) TF_LAMBDA_INLINE -> u32x4* {
            constexpr int b = decltype(Bc)::value;
            if constexpr (b == 0) return s0;
            else if constexpr (b == 1) return s1;
            else if constexpr (b == 2) return s2;
            else if constexpr (b == 3) return s3;
            else return s4;
        };
        auto buf_b = [&](auto Bc) TF_LAMBDA_INLINE -> u32x4* { return buf_a(Bc) + kDlVec; };
        // Loads of the walk's next block (byte offset = tile origin + k block
        // * k-block step within the batch element), then advance the walk.
        KWalk walk;
        walk.init(A, B, 2 * p.stride_a, 2 * p.stride_b, kb_beg, nk, kpb);
        const uint32_t ta0 = 2u * (A_KMAJ ? (uint32_t)m0 * (uint32_t)p.lda : (uint32_t)m0);
        const uint32_t tb0 = 2u * (B_KMAJ ? (uint32_t)n0 * (uint32_t)p.ldb : (uint32_t)n0);
        const uint32_t a_kstep = 2u * kDlK * (A_KMAJ ? 1u : (uint32_t)p.lda);
        const uint32_t b_kstep = 2u * kDlK * (B_KMAJ ? 1u : (uint32_t)p.ldb);
        const uint32_t wave_lds = dl_wave_offset<kDlLoads>();
        auto issue_next = [&](u32x4* la, u32x4* lb) TF_LAMBDA_INLINE {
            dl_issue(dl_rsrc(walk.a_base, p.a_bytes), ta0 + (uint32_t)walk.kin * a_kstep, voff_a,
                     lds_addr(la) + wave_lds);
            dl_issue(dl_rsrc(walk.b_base, p.b_bytes), tb0 + (uint32_t)walk.kin * b_kstep, voff_b,
                     lds_addr(lb) + wave_lds);
            walk.advance();
        };
        // Read order A0, B0..B3, A1..A3: the step's MFMAs (A_i x B_j,
        // i-major) can start after 2 reads, each further one needs at most
        // one more.
        auto read = [&](const u32x4* la, const u32x4* lb, int s, BigFrags& dst) TF_LAMBDA_INLINE {
            dst.a[0] = oa.frag(la, 0, s, half);
#pragma unroll
            for (int j = 0; j < 4; ++j) dst.b[j] = ob.frag(lb, j, s, half);
#pragma unroll
            for (int i = 1; i < 4; ++i) dst.a[i] = oa.frag(la, i, s, half);
        };
        constexpr int kReads = (A_KMAJ ? 4 : 8) + (B_KMAJ ? 4 : 8);  // LDS read instructions per k step
        // Every block but the last loads block t+5 (clamped to the last real
        // block: loads past the end land in buffers nobody reads again), so
        // exactly three blocks of loads are outstanding behind block t+1's
        // at each wait and all blocks have the same shape.  The last block
        // (no wait, barrier, loads or next-block reads) follows the loop.
        auto block = [&](auto Bc, int t) TF_LAMBDA_INLINE {
            constexpr int b = decltype(Bc)::value;
            u32x4* la = buf_a(Bc);
            u32x4* lb = buf_b(Bc);
            u32x4* na = buf_a(std::integral_constant<int, (b + 1) % kDlBufs>{});
            u32x4* nb = buf_b(std::integral_constant<int, (b + 1) % kDlBufs>{});
            read(la, lb, 1, f[1]);
            big_mfma(f[0], acc);
            static_for<8>([&](auto) TF_LAMBDA_INLINE {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);           // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, kReads / 8, 0);  // DS read
            });
            __builtin_amdgcn_sched_barrier(0);
            dl_barrier<3 * 2 * kDlLoads>();  // block t+1 has landed; block t fully read
            issue_next(la, lb);  // block min(t + kDlBufs, nk - 1)
            big_mfma_part<0, 4>(f[1], acc);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         // MFMA
            __builtin_amdgcn_sched_group_barrier(0x010, kDlLoads, 0);  // VMEM
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x010, kDlLoads, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_barrier(0);
            read(na, nb, 0, f[0]);
            big_mfma_part<4, 16>(f[1], acc);
            static_for<4>([&](auto) TF_LAMBDA_INLINE {
                __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);           // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, kReads / 4, 0);  // DS read
            });
            __builtin_amdgcn_sched_barrier(0);
        };
        // Prologue: blocks 0 .. 4 (clamped) into buffers 0 .. 4, wait for block 0.
        static_for<kDlBufs>([&](auto Bc) TF_LAMBDA_INLINE {
            issue_next(buf_a(Bc), buf_b(Bc));  // block min(Bc, nk - 1)
        });
        dl_barrier<(kDlBufs - 1) * 2 * kDlLoads>();  // block 0 has landed
        read(s0, s0 + kDlVec, 0, f[0]);
        // Blocks 0 .. nk-2, five per iteration (buffer = position in the group).
        int t = 0;
        bool stop = false;
        while (!stop) {
            static_for<kDlBufs>([&](auto Bc) TF_LAMBDA_INLINE {
                if (stop) return;
                if (t + 1 >= nk) {
                    stop = true;
                    return;
                }
                block(Bc, t);
                ++t;
            });
        }
        // Block nk-1: one copy with its buffer chosen at run time (five
        // unrolled copies, one per buffer, made the register allocator
        // spill accumulators around them).
        {
            const int rlast = t % kDlBufs;
            const u32x4* la = rlast == 0 ? s0 : rlast == 1 ? s1 : rlast == 2 ? s2 : rlast == 3 ? s3 : s4;
            read(la, la + kDlVec, 1, f[1]);
            big_mfma(f[0], acc);
            __builtin_amdgcn_sched_barrier(0);
            big_mfma(f[1], acc);
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // drain the clamped loads before the epilogue
    }
    __syncthreads();  // the epilogue stages through the ring buffers (one 32 KB buffer per wave)
    big_epilogue(p, acc, m0, n0, split, batch,
                 reinterpret_cast<float*>(wave == 0 ? s0 : wave == 1 ? s1 : wave == 2 ? s2 : s3));
}

// Eight-wave form of gemm_bf16_dl_kernel: the same 256 x 256 tile, LDS ring
// and pipeline, but 8 waves of 128 x 64 (two per SIMD, 128 accumulator
// registers each) so that one wave's stalls (barrier skew, fragment-read and
// scalar latency) can be covered by the other wave's MFMAs; each wave issues
// half as many direct loads.
// KTAIL: K % 64 != 0 (K % 8 == 0).  Each batch element spans 2 * ceil(K / 64)
// blocks of 32; the loads of k >= K get an offset past the descriptor and
// read zero (a compare and a select per load).
template <bool A_KMAJ, bool B_KMAJ, bool KTAIL = false>
__global__ __launch_bounds__(2 * kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_bf16_dl8_kernel(GemmParams p) {
    // One array per buffer (A block, then B block): the compiler tracks the
    // targets of in-flight LDS loads per LDS object and only for a few
    // objects; with more, every fragment read waits for all loads.
    __shared__ u32x4 s0[2 * kDlVec], s1[2 * kDlVec], s2[2 * kDlVec], s3[2 * kDlVec], s4[2 * kDlVec];

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int split = blockIdx.y;
    const int batch = blockIdx.z;
    const int m0 = tm * kBigTile, n0 = tn * kBigTile;
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A) + (int64_t)batch * p.stride_a;
    const uint16_t* B = reinterpret_cast<const uint16_t*>(p.B) + (int64_t)batch * p.stride_b;
    // Splits are counted in 64-deep blocks (the last one partly past K
    // with KTAIL): two of ours each.
    const int kb64_elem = KTAIL ? (p.K + 63) / 64 : p.K / 64;
    const int kb64_total = kb64_elem * p.reduce_batch;
    const int kb64_beg = split * p.kb_per_split;
    const int nk = 2 * max(0, min(kb64_total, kb64_beg + p.kb_per_split) - kb64_beg);
    const int kb_beg = 2 * kb64_beg;
    const int kpb = 2 * kb64_elem;  // 32-deep blocks per batch element

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int half = lane >> 5;
    v16f acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};

    if (nk > 0) {
        DlOperand<A_KMAJ> oa;
        DlOperand<B_KMAJ, 2> ob;
        oa.init((wave >> 2) * 128);
        ob.init((wave & 3) * 64);
        uint32_t voff_a[kDl8Loads], voff_b[kDl8Loads];
        dl_offsets<A_KMAJ, kDl8Loads>(p.lda, voff_a);
        dl_offsets<B_KMAJ, kDl8Loads>(p.ldb, voff_b);
        BigFrags8 f[2];
        auto buf_a = [&](auto Bc) TF_LAMBDA_INLINE -> u32x4* {
            constexpr int b = decltype(Bc)::value;
            if constexpr (b == 0) return s0;
            else if constexpr (b == 1) return s1;
            else if constexpr (b == 2) return s2;
            else if constexpr (b == 3) return s3;
            else return s4;
        };
        auto buf_b = [&](auto Bc) TF_LAMBDA_INLINE -> u32x4* { return buf_a(Bc) + kDlVec; };
        // Loads of the walk's next block (byte offset = tile origin + k block
        // * k-block step within the batch element), then advance the walk.
        KWalk walk;
        walk.init(A, B, 2 * p.stride_a, 2 * p.stride_b, kb_beg, nk, kpb);
        const uint32_t ta0 = 2u * (A_KMAJ ? (uint32_t)m0 * (uint32_t)p.lda : (uint32_t)m0);
        const uint32_t tb0 = 2u * (B_KMAJ ? (uint32_t)n0 * (uint32_t)p.ldb : (uint32_t)n0);
        const uint32_t a_kstep = 2u * kDlK * (A_KMAJ ? 1u : (uint32_t)p.lda);
        const uint32_t b_kstep = 2u * kDlK * (B_KMAJ ? 1u : (uint32_t)p.ldb);
        const uint32_t wave_lds = dl_wave_offset<kDl8Loads>();
        int kl_a[kDl8Loads], kl_b[kDl8Loads];
        if constexpr (KTAIL) {
            dl_klane<A_KMAJ, kDl8Loads>(kl_a);
            dl_klane<B_KMAJ, kDl8Loads>(kl_b);
        }
        auto issue_next = [&](u32x4* la, u32x4* lb) TF_LAMBDA_INLINE {
            const uint32_t so_a = ta0 + (uint32_t)walk.kin * a_kstep, so_b = tb0 + (uint32_t)walk.kin * b_kstep;
            if constexpr (KTAIL) {
                const int rem = p.K - walk.kin * kDlK;  // k of this block still inside K
                uint32_t va[kDl8Loads], vb[kDl8Loads];
#pragma unroll
                for (int i = 0; i < kDl8Loads; ++i) {
                    va[i] = kl_a[i] < rem ? voff_a[i] : kDlOob;
                    vb[i] = kl_b[i] < rem ? voff_b[i] : kDlOob;
                }
                dl_issue<kDl8Loads>(dl_rsrc(walk.a_base, p.a_bytes), so_a, va, lds_addr(la) + wave_lds);
                dl_issue<kDl8Loads>(dl_rsrc(walk.b_base, p.b_bytes), so_b, vb, lds_addr(lb) + wave_lds);
            } else {
                dl_issue<kDl8Loads>(dl_rsrc(walk.a_base, p.a_bytes), so_a, voff_a, lds_addr(la) + wave_lds);
                dl_issue<kDl8Loads>(dl_rsrc(walk.b_base, p.b_bytes), so_b, voff_b, lds_addr(lb) + wave_lds);
            }
            walk.advance();
        };
        // Read order A0, B0..B3, A1..A3: the step's MFMAs (A_i x B_j,
        // i-major) can start after 2 reads, each further one needs at most
        // one more.
        auto read = [&](const u32x4* la, const u32x4* lb, int s, BigFrags8& dst) TF_LAMBDA_INLINE {
            dst.a[0] = oa.frag(la, 0, s, half);
#pragma unroll
            for (int j = 0; j < 2; ++j) dst.b[j] = ob.frag(lb, j, s, half);
#pragma unroll
            for (int i = 1; i < 4; ++i) dst.a[i] = oa.frag(la, i, s, half);
        };
        constexpr int kReads = (A_KMAJ ? 4 : 8) + (B_KMAJ ? 2 : 4);  // LDS read instructions per k step
        // Every block but the last loads block t+5 (clamped to the last real
        // block: loads past the end land in buffers nobody reads again), so
        // exactly three blocks of loads are outstanding behind block t+1's
        // at each wait and all blocks have the same shape.  The last block
        // (no wait, barrier, loads or next-block reads) follows the loop.
        auto block = [&](auto Bc, int t) TF_LAMBDA_INLINE {
            constexpr int b = decltype(Bc)::value;
            u32x4* la = buf_a(Bc);
            u32x4* lb = buf_b(Bc);
            u32x4* na = buf_a(std::integral_constant<int, (b + 1) % kDlBufs>{});
            u32x4* nb = buf_b(std::integral_constant<int, (b + 1) % kDlBufs>{});
            read(la, lb, 1, f[1]);
            big_mfma8(f[0], acc);
            static_for<8>([&](auto) TF_LAMBDA_INLINE {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, (kReads + 7) / 8, 0);  // DS read
            });
            __builtin_amdgcn_sched_barrier(0);
            dl_barrier<3 * 2 * kDl8Loads>();  // block t+1 has landed; block t fully read
            issue_next(la, lb);  // block min(t + kDlBufs, nk - 1)
            big_mfma8_part<0, 2>(f[1], acc);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // MFMA
            __builtin_amdgcn_sched_group_barrier(0x010, kDl8Loads, 0);  // VMEM
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x010, kDl8Loads, 0);
            __builtin_amdgcn_sched_barrier(0);
            read(na, nb, 0, f[0]);
            big_mfma8_part<2, 8>(f[1], acc);
            static_for<6>([&](auto) TF_LAMBDA_INLINE {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, (kReads + 5) / 6, 0);  // DS read
            });
            __builtin_amdgcn_sched_barrier(0);
        };
        // Prologue: blocks 0 .. 4 (clamped) into buffers 0 .. 4, wait for block 0.
        static_for<kDlBufs>([&](auto Bc) TF_LAMBDA_INLINE {
            issue_next(buf_a(Bc), buf_b(Bc));  // block min(Bc, nk - 1)
        });
        dl_barrier<(kDlBufs - 1) * 2 * kDl8Loads>();  // block 0 has landed
        read(s0, s0 + kDlVec, 0, f[0]);
        // Blocks 0 .. nk-2, five per iteration (buffer = position in the group).
        int t = 0;
        bool stop = false;
        while (!stop) {
            static_for<kDlBufs>([&](auto Bc) TF_LAMBDA_INLINE {
                if (stop) return;
                if (t + 1 >= nk) {
                    stop = true;
                    return;
                }
                block(Bc, t);
                ++t;
            });
        }
        // Block nk-1: one copy with its buffer chosen at run time (five
        // unrolled copies, one per buffer, made the register allocator
        // spill accumulators around them).
        {
            const int rlast = t % kDlBufs;
            const u32x4* la = rlast == 0 ? s0 : rlast == 1 ? s1 : rlast == 2 ? s2 : rlast == 3 ? s3 : s4;
            read(la, la + kDlVec, 1, f[1]);
            big_mfma8(f[0], acc);
            __builtin_amdgcn_sched_barrier(0);
            big_mfma8(f[1], acc);
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // drain the clamped loads before the epilogue
    }
    __syncthreads();  // the epilogue stages through the ring buffers (one 32 KB buffer per wave)
    // 64 x 64 floats (16 KB) of staging per wave: waves 2b, 2b + 1 share buffer b.
    u32x4* sb = (wave >> 1) == 0 ? s0 : (wave >> 1) == 1 ? s1 : (wave >> 1) == 2 ? s2 : s3;
    big_epilogue<64>(p, acc, m0, n0, split, batch, reinterpret_cast<float*>(sb) + (wave & 1) * 4096);
}

// Eight waves in two groups of four, one wave of each group per SIMD, with
// their phases offset by half a block ("ping-pong"): while one group runs
// a block's 16 MFMAs from registers, the other issues its share of a later
// block's direct loads and reads the next block's fragments from LDS, then
// they swap, so each SIMD's MFMA pipe is fed by one of its two waves while
// the other waits (for LDS reads, for loads, at the barrier).  Same tile,
// wave layout, LDS ring (five 32-deep blocks), loads, fragments and
// epilogue as gemm_bf16_dl8_kernel.
//
// Every wave runs the same loop: for block t, M(t) (issue its share of
// block t+4 into block t-1's buffer when t >= 1, read block t's fragments),
// barrier, C(t) (16 MFMAs), barrier.  Group 1 passes one extra barrier before
// the loop and group 0 one after it, so when group 0 is in M(t) group 1 is
// in C(t-1), and when group 0 is in C(t) group 1 is in M(t).  Every barrier
// waits (in each wave) for all of the wave's loads but its newest three
// blocks and for its LDS reads.  Hazards: block t is read in M(t) by group 0
// (phase 2t) and group 1 (phase 2t+1); a wave's share of block t is waited
// for before the barrier that opens phase 2t (it was issued three or more
// blocks earlier); block t-1's buffer is refilled in M(t), from phase 2t
// on, after both groups have read it (phases 2t-2 and 2t-1).
template <bool A_KMAJ, bool B_KMAJ, bool KTAIL = false>
__global__ __launch_bounds__(2 * kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_bf16_pp_kernel(GemmParams p) {
    __shared__ u32x4 s0[2 * kDlVec], s1[2 * kDlVec], s2[2 * kDlVec], s3[2 * kDlVec], s4[2 * kDlVec];

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int split = blockIdx.y;
    const int batch = blockIdx.z;
    const int m0 = tm * kBigTile, n0 = tn * kBigTile;
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A) + (int64_t)batch * p.stride_a;
    const uint16_t* B = reinterpret_cast<const uint16_t*>(p.B) + (int64_t)batch * p.stride_b;
    const int kb64_elem = KTAIL ? (p.K + 63) / 64 : p.K / 64;
    const int kb64_total = kb64_elem * p.reduce_batch;
    const int kb64_beg = split * p.kb_per_split;
    const int nk = 2 * max(0, min(kb64_total, kb64_beg + p.kb_per_split) - kb64_beg);
    const int kb_beg = 2 * kb64_beg;
    const int kpb = 2 * kb64_elem;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int half = lane >> 5;
    const bool g1 = __builtin_amdgcn_readfirstlane(wave >> 2) != 0;  // wave-uniform
    v16f acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};

    if (nk > 0) {
        DlOperand<A_KMAJ> oa;
        DlOperand<B_KMAJ, 2> ob;
        oa.init((wave >> 2) * 128);
        ob.init((wave & 3) * 64);
        uint32_t voff_a[kDl8Loads], voff_b[kDl8Loads];
        dl_offsets<A_KMAJ, kDl8Loads>(p.lda, voff_a);
        dl_offsets<B_KMAJ, kDl8Loads>(p.ldb, voff_b);
        BigFrags8 f[2];
        auto buf_a = [&](auto Bc) TF_LAMBDA_INLINE -> u32x4* {
            constexpr int b = decltype(Bc)::value;
            if constexpr (b == 0) return s0;
            else if constexpr (b == 1) return s1;
            else if constexpr (b == 2) return s2;
            else if constexpr (b == 3) return s3;
            else return s4;
        };
        auto buf_b = [&](auto Bc) TF_LAMBDA_INLINE -> u32x4* { return buf_a(Bc) + kDlVec; };
        KWalk walk;
        walk.init(A, B, 2 * p.stride_a, 2 * p.stride_b, kb_beg, nk, kpb);
        const uint32_t ta0 = 2u * (A_KMAJ ? (uint32_t)m0 * (uint32_t)p.lda : (uint32_t)m0);
        const uint32_t tb0 = 2u * (B_KMAJ ? (uint32_t)n0 * (uint32_t)p.ldb : (uint32_t)n0);
        const uint32_t a_kstep = 2u * kDlK * (A_KMAJ ? 1u : (uint32_t)p.lda);
        const uint32_t b_kstep = 2u * kDlK * (B_KMAJ ? 1u : (uint32_t)p.ldb);
        const uint32_t wave_lds = dl_wave_offset<kDl8Loads>();
        int kl_a[kDl8Loads], kl_b[kDl8Loads];
        if constexpr (KTAIL) {
            dl_klane<A_KMAJ, kDl8Loads>(kl_a);
            dl_klane<B_KMAJ, kDl8Loads>(kl_b);
        }
        auto issue_next = [&](u32x4* la, u32x4* lb) TF_LAMBDA_INLINE {
            const uint32_t so_a = ta0 + (uint32_t)walk.kin * a_kstep, so_b = tb0 + (uint32_t)walk.kin * b_kstep;
            if constexpr (KTAIL) {
                const int rem = p.K - walk.kin * kDlK;
                uint32_t va[kDl8Loads], vb[kDl8Loads];
#pragma unroll
                for (int i = 0; i < kDl8Loads; ++i) {
                    va[i] = kl_a[i] < rem ? voff_a[i] : kDlOob;
                    vb[i] = kl_b[i] < rem ? voff_b[i] : kDlOob;
                }
                dl_issue<kDl8Loads>(dl_rsrc(walk.a_base, p.a_bytes), so_a, va, lds_addr(la) + wave_lds);
                dl_issue<kDl8Loads>(dl_rsrc(walk.b_base, p.b_bytes), so_b, vb, lds_addr(lb) + wave_lds);
            } else {
                dl_issue<kDl8Loads>(dl_rsrc(walk.a_base, p.a_bytes), so_a, voff_a, lds_addr(la) + wave_lds);
                dl_issue<kDl8Loads>(dl_rsrc(walk.b_base, p.b_bytes), so_b, voff_b, lds_addr(lb) + wave_lds);
            }
            walk.advance();
        };
        // Both k steps of a block: A0, B0, B1, A1..A3 per step.
        auto read_block = [&](const u32x4* la, const u32x4* lb) TF_LAMBDA_INLINE {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                f[s].a[0] = oa.frag(la, 0, s, half);
#pragma unroll
                for (int j = 0; j < 2; ++j) f[s].b[j] = ob.frag(lb, j, s, half);
#pragma unroll
                for (int i = 1; i < 4; ++i) f[s].a[i] = oa.frag(la, i, s, half);
            }
        };
        constexpr int kAhead = 3 * 2 * kDl8Loads;  // loads of the newest three blocks
        // Prologue: blocks 0 .. 4 (clamped) into buffers 0 .. 4.
        static_for<kDlBufs>([&](auto Bc) TF_LAMBDA_INLINE { issue_next(buf_a(Bc), buf_b(Bc)); });
        dl_barrier<(kDlBufs - 1) * 2 * kDl8Loads>();  // block 0 has landed
        if (g1) dl_barrier<kAhead>();                 // group 1 starts half a block later
        int t = 0;
        bool stop = false;
        while (!stop) {
            static_for<kDlBufs>([&](auto Bc) TF_LAMBDA_INLINE {
                constexpr int bp = (decltype(Bc)::value + kDlBufs - 1) % kDlBufs;
                if (stop) return;
                // M(t)
                if (t >= 1) issue_next(buf_a(std::integral_constant<int, bp>{}), buf_b(std::integral_constant<int, bp>{}));
                read_block(buf_a(Bc), buf_b(Bc));
                __builtin_amdgcn_sched_barrier(0);
                // Group 1's share of block t+1 is read by group 0 right after
                // this barrier; group 0's is not needed until the next one.
                if (g1) dl_barrier<kAhead>();
                else dl_barrier<kAhead + 2 * kDl8Loads>();
                // C(t)
                big_mfma8(f[0], acc);
                big_mfma8(f[1], acc);
                __builtin_amdgcn_sched_barrier(0);
                dl_barrier<kAhead>();
                ++t;
                if (t >= nk) stop = true;
            });
        }
        if (!g1) dl_barrier<kAhead>();  // matches group 1's extra barrier
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // drain the clamped loads before the epilogue
    }
    __syncthreads();
    u32x4* sb = (wave >> 1) == 0 ? s0 : (wave >> 1) == 1 ? s1 : (wave >> 1) == 2 ? s2 : s3;
    big_epilogue<64>(p, acc, m0, n0, split, batch, reinterpret_cast<float*>(sb) + (wave & 1) * 4096);
}

// Edge-tile kernel (or every tile when the direct path does not apply):
// register-staged, bounds-checked 64-deep blocks over the tiles edge_coords
// assigns.
template <bool A_KMAJ, bool B_KMAJ>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_big_kernel(GemmParams p) {
    __shared__ u32x4 lds_a0[kBigTile * 8], lds_a1[kBigTile * 8];
    __shared__ u32x4 lds_b0[kBigTile * 8], lds_b1[kBigTile * 8];

    int tm, tn;
    edge_coords(p, tm, tn);
    const int split = blockIdx.y;
    const int batch = blockIdx.z;
    const int m0 = tm * kBigTile, n0 = tn * kBigTile;
    const int kb_total = ((p.K + kBigK - 1) / kBigK) * p.reduce_batch;
    const int kb_beg = split * p.kb_per_split;
    const int nk = max(0, min(kb_total, kb_beg + p.kb_per_split) - kb_beg);
    big_tile_guarded<A_KMAJ, B_KMAJ>(p, m0, n0, split, batch, kb_beg, nk, lds_a0, lds_a1, lds_b0, lds_b1);
}

// ---------------------------------------------------------------------------
// fp32 kernel: 128 x BN x 32 per 256-thread workgroup (BN = 128, or 64 for
// grids that would leave CUs idle), 4 waves in 2 x 2, each 64 x BN/2 =
// 2 x NSUB accumulators of v_mfma_f32_32x32x2_f32.
//
// Both operands are staged K-major in LDS ([rows][32 + 4] floats: with the
// 4-float pad the rows of a b128 fragment read hit distinct banks); an
// MN-major operand is transposed in registers in 4 x 4 blocks while staged.
// Lane half h feeds k = 16h + s to the s-th MFMA of a block (the sum order
// within a block is permuted; the reference's sequential loop,
// tensor/Tensor.cpp:356-360, differs only by rounding), so one b128 read
// gives a lane four consecutive steps ("a quad").
//
// Pipeline (three LDS stages, one barrier per 32-deep block): while block k
// is multiplied out of stage k%3, the registers holding block k+2 are written
// to stage (k+2)%3, the global loads of block k+3 are issued into those
// registers, and the first fragments of block k+1 (stage (k+1)%3, written a
// block earlier) are read before the barrier, so no LDS latency follows it.
// Loads past the last block are clamped to it (their writes land in a stage
// nobody reads again).  Interior tiles take an unguarded load path with the
// memory operations pinned between the MFMAs (sched_group_barrier); edge
// tiles a bounds-checked one with zero fill (separate instantiations).
// ---------------------------------------------------------------------------
constexpr int kF32K = 32;
constexpr int kF32LD = kF32K + 4;
constexpr int kF32Stages = 3;

template <int ROWS, bool KMAJ, bool GUARD>
struct F32Stage {
    // K-major: vector i of thread t is row t/8 + 32i, k 4(t%8) .. +3 (a
    // wave's 8-lane groups read 128 contiguous bytes of one row).
    // MN-major: thread t < 8 * ROWS/4 owns the 4 x 4 block (k 4kb .. +3,
    // rows 4mb .. +3); reg[kk] holds k row 4kb + kk.  Lanes 4i .. 4i+3 take
    // consecutive mb (64 contiguous bytes of a k row) and the next four lanes
    // the next kb, so a load reads whole 16 * ROWS-byte k rows, and the 8
    // lanes of a group store at 8 distinct 16-byte bank groups (rows 4 apart
    // are 144 words apart: 4 groups by mb, times 2 by kb).
    static constexpr int NK = ROWS / 32;  // K-major 16-byte vectors per thread
    static constexpr int NB = 8 * (ROWS / 4);  // MN-major blocks (threads with work)
    static constexpr int N4 = KMAJ ? NK : 4;
    static constexpr int MH = ROWS / 16;  // groups of 4 mb
    f32x4 reg[N4];

    __device__ __forceinline__ static void mn_block(int t, int& mb, int& kb) {
        const int rest = t >> 3;
        mb = (t & 3) + 4 * (rest % MH);
        kb = ((t >> 2) & 1) + 2 * (rest / MH);
    }

    __device__ __forceinline__ static f32x4 load4(const float* __restrict__ p, int n, bool vec) {
        if (!GUARD || (vec && n >= 4)) return *reinterpret_cast<const f32x4*>(p);
        return f32x4{n > 0 ? p[0] : 0.0f, n > 1 ? p[1] : 0.0f, n > 2 ? p[2] : 0.0f, n > 3 ? p[3] : 0.0f};
    }

    __device__ __forceinline__ void load(const float* __restrict__ p, int64_t ld, int row0, int rows, int k0, int kend,
                                         bool vec) {
        const int t = threadIdx.x;
        if (KMAJ) {
            const int c = t & 7, r = t >> 3;
            static_for<NK>([&](auto I) TF_LAMBDA_INLINE {
                constexpr int i = decltype(I)::value;
                const int row = row0 + r + 32 * i, k = k0 + 4 * c;
                const float* src = p + (int64_t)row * ld + k;
                if (!GUARD) reg[i] = *reinterpret_cast<const f32x4*>(src);
                else reg[i] = row < rows ? load4(src, kend - k, vec) : f32x4{0.f, 0.f, 0.f, 0.f};
            });
        } else {
            if (NB < kThreads && t >= NB) return;
            int mb, kb;
            mn_block(t, mb, kb);
            const int m = row0 + 4 * mb;
            static_for<4>([&](auto KK) TF_LAMBDA_INLINE {
                constexpr int kk = decltype(KK)::value;
                const int k = k0 + 4 * kb + kk;
                const float* src = p + (int64_t)k * ld + m;
                if (!GUARD) reg[kk] = *reinterpret_cast<const f32x4*>(src);
                else reg[kk] = k < kend ? load4(src, rows - m, vec) : f32x4{0.f, 0.f, 0.f, 0.f};
            });
        }
    }

    __device__ __forceinline__ void store(float* __restrict__ lds) const {
        const int t = threadIdx.x;
        if (KMAJ) {
            const int c = t & 7, r = t >> 3;
            static_for<NK>([&](auto I) TF_LAMBDA_INLINE {
                constexpr int i = decltype(I)::value;
                *reinterpret_cast<f32x4*>(lds + (r + 32 * i) * kF32LD + 4 * c) = reg[i];
            });
        } else {
            if (NB < kThreads && t >= NB) return;
            int mb, kb;
            mn_block(t, mb, kb);
            // Row 4mb + j of the tile gets k 4kb .. +3 = element j of reg[0..3].
            static_for<4>([&](auto J) TF_LAMBDA_INLINE {
                constexpr int j = decltype(J)::value;
                *reinterpret_cast<f32x4*>(lds + (4 * mb + j) * kF32LD + 4 * kb) =
                    f32x4{reg[0][j], reg[1][j], reg[2][j], reg[3][j]};
            });
        }
    }
};

template <int BN, bool A_KMAJ, bool B_KMAJ, bool GUARD>
__device__ __forceinline__ void f32_tile(const GemmParams& p, int m0, int n0, int split, int batch, int kb_beg, int nk,
                                         float* lds) {
    constexpr int WN = BN / 2;
    constexpr int NSUB = WN / 32;
    constexpr int A_SZ = BM * kF32LD;          // floats of A per stage
    constexpr int STAGE = (BM + BN) * kF32LD;  // floats per stage
    const float* A = reinterpret_cast<const float*>(p.A) + (int64_t)batch * p.stride_a;
    const float* B = reinterpret_cast<const float*>(p.B) + (int64_t)batch * p.stride_b;
    const int kb_per_b = (p.K + kF32K - 1) / kF32K;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l32 = lane & 31;

    v16f acc[2][NSUB];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NSUB; ++j) acc[i][j] = v16f{};

    if (nk > 0) {
        F32Stage<BM, A_KMAJ, GUARD> sa;
        F32Stage<BN, B_KMAJ, GUARD> sb;
        // Fragments of one quad (4 k steps): A sub-tiles 0,1 and B sub-tiles.
        struct Quad {
            f32x4 a[2], b[NSUB];
        };
        Quad f[2];
        const int a_off = (wm * 64 + l32) * kF32LD + 16 * half;
        const int b_off = A_SZ + (wn * WN + l32) * kF32LD + 16 * half;
        // Block k of this slice (clamped to the last one).
        auto load_block = [&](int k) TF_LAMBDA_INLINE {
            const int kb = kb_beg + min(k, nk - 1);
            const int b = kb / kb_per_b, k0 = (kb - b * kb_per_b) * kF32K;
            sa.load(A + (int64_t)b * p.stride_a, p.lda, m0, p.M, k0, p.K, p.vec_a);
            sb.load(B + (int64_t)b * p.stride_b, p.ldb, n0, p.N, k0, p.K, p.vec_b);
        };
        auto store_block = [&](float* st) TF_LAMBDA_INLINE {
            sa.store(st);
            sb.store(st + A_SZ);
        };
        auto read = [&](const float* st, int q, Quad& d) TF_LAMBDA_INLINE {
#pragma unroll
            for (int i = 0; i < 2; ++i) d.a[i] = *reinterpret_cast<const f32x4*>(st + a_off + 32 * i * kF32LD + 4 * q);
#pragma unroll
            for (int j = 0; j < NSUB; ++j)
                d.b[j] = *reinterpret_cast<const f32x4*>(st + b_off + 32 * j * kF32LD + 4 * q);
        };
        auto mfma_quad = [&](const Quad& d) TF_LAMBDA_INLINE {
            static_for<4>([&](auto S) TF_LAMBDA_INLINE {
                constexpr int s = decltype(S)::value;
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < NSUB; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(d.a[i][s], d.b[j][s], acc[i][j], 0, 0, 0);
            });
        };
        constexpr int kMf = 4 * 2 * NSUB;  // MFMAs per quad
        constexpr int kRd = 2 + NSUB;      // LDS reads per quad
        // Interleave the quad's MFMAs with the kRd fragment reads issued
        // before them (plus, in the first quad, the stage writes and loads).
        auto pin_reads = [&]() TF_LAMBDA_INLINE {
            static_for<kRd>([&](auto) TF_LAMBDA_INLINE {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            });
        };
        constexpr int kWr = F32Stage<BM, A_KMAJ, GUARD>::N4 + F32Stage<BN, B_KMAJ, GUARD>::N4;  // stage writes per thread
        constexpr bool kPinStage = !GUARD && F32Stage<BN, B_KMAJ, GUARD>::NB >= kThreads;

        // Prologue: blocks 0 and 1 into stages 0 and 1, block 2 into registers.
        load_block(0);
        store_block(lds);
        load_block(1);
        store_block(lds + STAGE);
        load_block(2);
        dl_barrier<63>();
        read(lds, 0, f[0]);
        uint32_t s0 = 0, s1 = STAGE, s2 = 2 * STAGE;  // stage offsets of blocks k, k+1, k+2
        for (int k = 0; k < nk; ++k) {
            const float* cur = lds + s0;
            // Quad 0: reads of quad 1, block k+2 to its stage, loads of block k+3.
            read(cur, 1, f[1]);
            store_block(lds + s2);
            load_block(k + 3);
            mfma_quad(f[0]);
            if constexpr (kPinStage) {
                pin_reads();
                static_for<kWr / 2>([&](auto) TF_LAMBDA_INLINE {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);  // DS write
                });
                static_for<kWr / 2>([&](auto) TF_LAMBDA_INLINE {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // VMEM read
                });
            }
            __builtin_amdgcn_sched_barrier(0);
            // Quads 1 .. 3: each reads the fragments of the next quad; quad 3
            // those of block k+1's quad 0.
            read(cur, 2, f[0]);
            mfma_quad(f[1]);
            if constexpr (!GUARD) pin_reads();
            __builtin_amdgcn_sched_barrier(0);
            read(cur, 3, f[1]);
            mfma_quad(f[0]);
            if constexpr (!GUARD) pin_reads();
            __builtin_amdgcn_sched_barrier(0);
            read(lds + s1, 0, f[0]);
            mfma_quad(f[1]);
            if constexpr (!GUARD) pin_reads();
            __builtin_amdgcn_sched_barrier(0);
            // Block k+2's stage written and block k's stage fully read.
            dl_barrier<63>();
            const uint32_t t = s0;
            s0 = s1;
            s1 = s2;
            s2 = t;
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // drain the clamped loads
    }
    store_wave<NSUB, false, false>(p, acc, m0 + wm * 64, n0 + wn * WN, (int64_t)batch * p.stride_c, split);
}

template <int BN, bool A_KMAJ, bool B_KMAJ>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) float lds[kF32Stages * (BM + BN) * kF32LD];
    int tm, tn;
    edge_coords(p, tm, tn);
    const int split = blockIdx.y;
    const int batch = blockIdx.z;
    const int m0 = tm * BM, n0 = tn * BN;
    const int kb_per_b = (p.K + kF32K - 1) / kF32K;
    const int kb_total = kb_per_b * p.reduce_batch;
    const int kb_beg = split * p.kb_per_split;
    const int nk = max(0, min(kb_total, kb_beg + p.kb_per_split) - kb_beg);
    const bool interior = p.vec_a && p.vec_b && m0 + BM <= p.M && n0 + BN <= p.N && p.K % kF32K == 0;
    if (interior)
        f32_tile<BN, A_KMAJ, B_KMAJ, false>(p, m0, n0, split, batch, kb_beg, nk, lds);
    else
        f32_tile<BN, A_KMAJ, B_KMAJ, true>(p, m0, n0, split, batch, kb_beg, nk, lds);
}

// ---------------------------------------------------------------------------
// fp32 direct-to-LDS kernel (tiles inside an int_m x int_n grid of 128 x 128,
// K % 32 == 0, 16-byte loadable operands): the global loads write LDS
// directly (buffer_load_dwordx4 ... lds, as in the bf16 direct kernel), so no
// staging registers and no LDS stores; block k's loads are issued two blocks
// ahead into a four-stage ring (128 KB).
//
// 512 threads: waves w and w + 4 share the 64 x 64 output block w & 3 (2 x 2
// sub-tiles of v_mfma_f32_32x32x2_f32) and split every 32-deep block: group
// g = w / 4 takes quads 2g and 2g + 1 (lane half h feeds k = 16h + 4q + s at
// step s of quad q, the k order of the register-staged kernel).  Two waves
// per SIMD keep its matrix core busy through each other's barrier and LDS
// waits.  At the end each pair adds its halves through LDS (own + partner:
// the same sum in both waves, fp addition commutes) and each wave stores one
// 32-row sub-tile of the block.
//
// LDS layout per operand block (16 KB, written 1 KB per load instruction):
//   K-major  [128 rows][8 chunks of 4 k]; chunk c of row r sits in slot
//            c ^ f32dl_swz(r), so the b128 fragment reads of 16 consecutive
//            rows hit 16 distinct 4-bank groups (rows 2 apart share banks);
//   MN-major [32 k][128 rows], as in memory; a lane reads the row pair
//            2c, 2c + 1 of one k with one ds_read_b64, so sub-tile 0 of a
//            wave holds its rows 2c and sub-tile 1 its rows 2c + 1 (the
//            epilogue writes those rows / columns interleaved).
// ---------------------------------------------------------------------------
constexpr int kF32DlThreads = 512;
constexpr int kF32DlStages = 4;
constexpr int kF32DlOp = BM * kF32K;                                     // floats of one operand block
constexpr int kF32DlLoads = kF32DlOp * 4 / 1024 / (kF32DlThreads / 64);  // 1 KB loads per wave per block

__device__ __forceinline__ int f32dl_swz(int row) { return (row >> 1) & 7; }

// Byte offsets (from the tile origin) of this lane's direct loads of one
// operand block; wave w fills 1 KB pieces kF32DlLoads*w .. of it.
template <bool KMAJ>
__device__ __forceinline__ void f32dl_offsets(int64_t ld, uint32_t (&voff)[kF32DlLoads]) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < kF32DlLoads; ++i) {
        const int blk = w * kF32DlLoads + i;
        if (KMAJ) {
            const int row = blk * 8 + (l >> 3);  // lane l fills slot l & 7 of row
            voff[i] = 4u * ((uint32_t)row * (uint32_t)ld + 4u * (uint32_t)((l & 7) ^ f32dl_swz(row)));
        } else {
            const int k = blk * 2 + (l >> 5);
            voff[i] = 4u * ((uint32_t)k * (uint32_t)ld + 4u * (uint32_t)(l & 31));
        }
    }
}

// Issue this wave's direct loads of one operand block (M0 = the 1 KB LDS
// destination; inline assembly for the reasons given at dl_issue).
// `lds_wave`: LDS byte address of this wave's first 1 KB of the block.
__device__ __forceinline__ void f32dl_issue(i32x4 rsrc, uint32_t tile_off, const uint32_t (&voff)[kF32DlLoads],
                                            uint32_t lds_wave) {
    static_for<kF32DlLoads>([&](auto I) TF_LAMBDA_INLINE {
        constexpr int i = decltype(I)::value;
        const uint32_t dst = lds_wave + i * 1024u;
        const uint32_t v = voff[i], so = tile_off;  // asm operands must be locals of the lambda
        const i32x4 r = rsrc;
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                     :
                     : "s"(dst), "v"(v), "s"(r), "s"(so)
                     : "memory", "m0");
    });
}

// One quad's fragments of one operand: the value of sub-tile i at step s.
template <bool KMAJ>
struct F32DlFrag;
template <>
struct F32DlFrag<true> {
    f32x4 v[2];
    __device__ __forceinline__ float at(int i, int s) const { return v[i][s]; }
};
template <>
struct F32DlFrag<false> {
    f32x2 v[4];
    __device__ __forceinline__ float at(int i, int s) const { return v[s][i]; }
};

// Per-lane LDS word offsets of one operand's fragment reads (wave rows
// wbase .. wbase + 63, quads 2g + qq).  K-major: sub-tile i's row for quad
// qq (swizzled chunk 4h + 2g + qq).  MN-major: the lane's row pair in k row
// 16h + 8g.
template <bool KMAJ>
struct F32DlOperand {
    int off[KMAJ ? 4 : 1];
    __device__ __forceinline__ void init(int wbase, int g) {
        const int l = threadIdx.x & 63, h = l >> 5, l32 = l & 31;
        if constexpr (KMAJ) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wbase + 32 * i + l32;
#pragma unroll
                for (int qq = 0; qq < 2; ++qq)
                    off[2 * i + qq] = r * kF32K + 4 * ((4 * h + 2 * g + qq) ^ f32dl_swz(r));
            }
        } else {
            off[0] = (16 * h + 8 * g) * BM + wbase + 2 * l32;
        }
    }
    __device__ __forceinline__ void read(const float* op, int qq, F32DlFrag<KMAJ>& d) const {
        if constexpr (KMAJ) {
#pragma unroll
            for (int i = 0; i < 2; ++i) d.v[i] = *reinterpret_cast<const f32x4*>(op + off[2 * i + qq]);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) d.v[s] = *reinterpret_cast<const f32x2*>(op + off[0] + (4 * qq + s) * BM);
        }
    }
};

constexpr int kF32DlPairFloats = 8 * 8 * 64 * 4;  // LDS floats of the pair reduction (8 KB per wave)

// Epilogue of the direct fp32 kernel for interior blocks without beta * C or
// a row bias.  The wave's 32 x 64 block (sub-tile row block g after the pair
// reduction) is staged in its own 8 KB of LDS (`stage`, 32 rows x 64
// floats) and written by whole rows: a lane takes 4 consecutive columns
// (16-byte stores; 16 lanes per row, 4 rows per pass), the pointer advances
// by 4 staged rows per pass, and the output form (OUT 0: split-K partial,
// 1: bf16, 2: fp32) and transform (XF 0: copy, 1: alpha * v + bias, 2: the
// same then ReLU) are fixed at compile time.  Writing element by element
// (store_wave) spends more time on address arithmetic and checks than on the
// stores.  Staged row rl of block g is row rl (A_PAIR: 2 rl + g; otherwise
// 32 g + rl) of the wave block; its column c is column c of the wave block
// (B_PAIR: accumulator j holds columns 2 l + j, so a lane's pair of
// accumulators is one 8-byte LDS write).  Returns false, having written
// nothing, when the block does not qualify.
template <bool A_PAIR, bool B_PAIR>
__device__ __forceinline__ bool f32dl_store_fast(const GemmParams& p, const v16f (&acc)[2][2], int g, int m_base,
                                                 int n_base, int64_t boff, int split, float* __restrict__ stage) {
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    float* part = p.partial ? p.partial + (int64_t)split * p.M * p.N : nullptr;
    if (!part && (p.beta != 0.0f || (has_bias && p.row_bias))) return false;
    if (part ? p.N % 4 != 0 : p.vec_c4 == 0) return false;
    if (m_base + 64 > p.M || n_base + 64 > p.N) return false;
    const int lane = threadIdx.x & 63, l32 = lane & 31, half = lane >> 5;
    // The kept block, chosen by value: indexing acc with the run-time g
    // (even under a branch per candidate) made the compiler keep all
    // accumulators in scratch memory.
    const v16f k0 = g ? acc[1][0] : acc[0][0];
    const v16f k1 = g ? acc[1][1] : acc[0][1];
    static_for<16>([&](auto R) TF_LAMBDA_INLINE {
        constexpr int r = decltype(R)::value;
        float* row = stage + (8 * (r >> 2) + 4 * half + (r & 3)) * 64;
        if constexpr (B_PAIR) {
            *reinterpret_cast<f32x2*>(row + 2 * l32) = f32x2{k0[r], k1[r]};
        } else {
            row[l32] = k0[r];
            row[32 + l32] = k1[r];
        }
    });
    const int rsub = lane >> 4, c4 = 4 * (lane & 15);
    const int col = n_base + c4;
    float cb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) cb[e] = has_bias ? p.bias[col + e] : 0.0f;
    const float alpha = p.alpha;
    const int row_step = A_PAIR ? 2 : 1;  // rows of C per staged row
    const int row0 = m_base + (A_PAIR ? g : 32 * g) + row_step * rsub;
    const float* src = stage + rsub * 64 + c4;
    auto copy = [&](auto OUT, auto XF) TF_LAMBDA_INLINE {
        constexpr int out = decltype(OUT)::value, xf = decltype(XF)::value;
        using Dst = std::conditional_t<out == 1, uint16_t, float>;
        const int64_t ld = out == 0 ? (int64_t)p.N : (int64_t)p.ldc;
        Dst* dst = out == 0 ? reinterpret_cast<Dst*>(part) + (int64_t)row0 * ld + col
                            : reinterpret_cast<Dst*>(p.C) + boff + (int64_t)row0 * ld + col;
#pragma unroll
        for (int pass = 0; pass < 8; ++pass) {
            f32x4 o = *reinterpret_cast<const f32x4*>(src + pass * 4 * 64);
            if constexpr (xf != 0) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float t = alpha * o[e] + cb[e];
                    o[e] = xf == 2 ? fmaxf(t, 0.0f) : t;
                }
            }
            if constexpr (out == 1)
                *reinterpret_cast<uint2*>(dst) = make_uint2(tfd::bf16x2_rne(o[0], o[1]), tfd::bf16x2_rne(o[2], o[3]));
            else
                *reinterpret_cast<f32x4*>(dst) = o;
            dst += 4 * row_step * ld;
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    const bool plain = alpha == 1.0f && !has_bias && !relu;
    if (part) copy(I0{}, I0{});
    else if (p.out_bf16) {
        if (plain) copy(I1{}, I0{});
        else if (relu) copy(I1{}, I2{});
        else copy(I1{}, I1{});
    } else {
        if (plain) copy(I2{}, I0{});
        else if (relu) copy(I2{}, I2{});
        else copy(I2{}, I1{});
    }
    return true;
}

template <bool A_KMAJ, bool B_KMAJ>
__global__ __launch_bounds__(kF32DlThreads) void gemm_f32_dl_kernel(GemmParams p) {
    constexpr int S = kF32DlStages;
    __shared__ __attribute__((aligned(16))) float lds[S * 2 * kF32DlOp];
    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int split = blockIdx.y;
    const int batch = blockIdx.z;
    const int m0 = tm * BM, n0 = tn * BM;
    const int kpb = p.K / kF32K;
    const int kb_total = kpb * p.reduce_batch;
    const int kb_beg = split * p.kb_per_split;
    const int nk = max(0, min(kb_total, kb_beg + p.kb_per_split) - kb_beg);
    const float* A = reinterpret_cast<const float*>(p.A) + (int64_t)batch * p.stride_a;
    const float* B = reinterpret_cast<const float*>(p.B) + (int64_t)batch * p.stride_b;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = wave >> 2, wm = (wave >> 1) & 1, wn = wave & 1;

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};

    if (nk > 0) {
        F32DlOperand<A_KMAJ> oa;
        F32DlOperand<B_KMAJ> ob;
        oa.init(wm * 64, g);
        ob.init(wn * 64, g);
        uint32_t voff_a[kF32DlLoads], voff_b[kF32DlLoads];
        f32dl_offsets<A_KMAJ>(p.lda, voff_a);
        f32dl_offsets<B_KMAJ>(p.ldb, voff_b);
        struct Quad {
            F32DlFrag<A_KMAJ> a;
            F32DlFrag<B_KMAJ> b;
        };
        Quad f[2];
        auto stage_a = [&](int st) TF_LAMBDA_INLINE { return lds + st * 2 * kF32DlOp; };
        // Loads of the walk's next block into stage st, then advance the walk.
        KWalk walk;
        walk.init(A, B, 4 * p.stride_a, 4 * p.stride_b, kb_beg, nk, kpb);
        const uint32_t ta0 = 4u * (A_KMAJ ? (uint32_t)m0 * (uint32_t)p.lda : (uint32_t)m0);
        const uint32_t tb0 = 4u * (B_KMAJ ? (uint32_t)n0 * (uint32_t)p.ldb : (uint32_t)n0);
        const uint32_t a_kstep = 4u * kF32K * (A_KMAJ ? 1u : (uint32_t)p.lda);
        const uint32_t b_kstep = 4u * kF32K * (B_KMAJ ? 1u : (uint32_t)p.ldb);
        const uint32_t wave_lds = lds_addr(lds) + dl_wave_offset<kF32DlLoads>();
        auto issue_next = [&](int st) TF_LAMBDA_INLINE {
            const uint32_t dst = wave_lds + (uint32_t)(st * 2 * kF32DlOp * 4);
            f32dl_issue(dl_rsrc(walk.a_base, p.a_bytes), ta0 + (uint32_t)walk.kin * a_kstep, voff_a, dst);
            f32dl_issue(dl_rsrc(walk.b_base, p.b_bytes), tb0 + (uint32_t)walk.kin * b_kstep, voff_b,
                        dst + kF32DlOp * 4);
            walk.advance();
        };
        auto read = [&](int st, int qq, Quad& d) TF_LAMBDA_INLINE {
            oa.read(stage_a(st), qq, d.a);
            ob.read(stage_a(st) + kF32DlOp, qq, d.b);
        };
        auto mfma_quad = [&](const Quad& d) TF_LAMBDA_INLINE {
            static_for<4>([&](auto Sc) TF_LAMBDA_INLINE {
                constexpr int s = decltype(Sc)::value;
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(d.a.at(i, s), d.b.at(j, s), acc[i][j], 0, 0, 0);
            });
        };
        constexpr int kRd = (A_KMAJ ? 2 : 4) + (B_KMAJ ? 2 : 4);  // LDS reads per quad
        auto pin_reads = [&]() TF_LAMBDA_INLINE {
            static_for<kRd>([&](auto) TF_LAMBDA_INLINE {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            });
        };
        // Block t in stage b = t % S (this wave's two quads of it).  Every
        // block but the last waits for block t+1 (S-3 newer blocks of loads
        // stay in flight), which also guarantees every wave is done with block
        // t-1's stage, loads block t+S-1 (clamped to the last block: loads
        // past the end land in stages nobody reads again) into that stage and
        // reads block t+1's first fragments.  LAST: no next block.
        auto block = [&](auto Bc, int t, auto LAST) TF_LAMBDA_INLINE {
            constexpr int b = decltype(Bc)::value;
            constexpr bool last = decltype(LAST)::value;
            read(b, 1, f[1]);
            mfma_quad(f[0]);
            pin_reads();
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (!last) {
                dl_barrier<(S - 3) * 2 * kF32DlLoads>();
                issue_next((b + S - 1) % S);  // block min(t + S - 1, nk - 1)
                read((b + 1) % S, 0, f[0]);
            }
            mfma_quad(f[1]);
            if constexpr (!last) pin_reads();
            __builtin_amdgcn_sched_barrier(0);
        };
        // Prologue: blocks 0 .. S-2 (clamped) into stages 0 .. S-2, wait for block 0.
        static_for<S - 1>([&](auto Bc) TF_LAMBDA_INLINE {
            constexpr int b = decltype(Bc)::value;
            issue_next(b);  // block min(b, nk - 1)
        });
        dl_barrier<(S - 2) * 2 * kF32DlLoads>();
        read(0, 0, f[0]);
        // Blocks 0 .. nk-2, S per iteration (stage = position in the group).
        int t = 0;
        bool stop = false;
        while (!stop) {
            static_for<S>([&](auto Bc) TF_LAMBDA_INLINE {
                if (stop) return;
                if (t + 1 >= nk) {
                    stop = true;
                    return;
                }
                block(Bc, t, std::false_type{});
                ++t;
            });
        }
        // Block nk-1.
        const int rlast = t % S;
        static_for<S>([&](auto Bc) TF_LAMBDA_INLINE {
            if (rlast == decltype(Bc)::value) block(Bc, t, std::true_type{});
        });
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // drain the clamped loads
    }
    // Pair reduction through LDS: wave w hands sub-tile row block 1 - g to
    // wave w ^ 4 and keeps block g (8 KB per wave, 1 KB per vector).
    __syncthreads();  // every wave is done with the stages
    f32x4* x = reinterpret_cast<f32x4*>(lds);
    static_for<2>([&](auto I) TF_LAMBDA_INLINE {
        constexpr int i = decltype(I)::value;
        if (i == g) return;
        static_for<8>([&](auto V) TF_LAMBDA_INLINE {
            constexpr int v = decltype(V)::value, j = v >> 2, r = 4 * (v & 3);
            x[(wave * 8 + v) * 64 + lane] = f32x4{acc[i][j][r], acc[i][j][r + 1], acc[i][j][r + 2], acc[i][j][r + 3]};
        });
    });
    __syncthreads();
    static_for<2>([&](auto I) TF_LAMBDA_INLINE {
        constexpr int i = decltype(I)::value;
        if (i != g) return;
        static_for<8>([&](auto V) TF_LAMBDA_INLINE {
            constexpr int v = decltype(V)::value, j = v >> 2, r = 4 * (v & 3);
            const f32x4 y = x[((wave ^ 4) * 8 + v) * 64 + lane];
            acc[i][j][r] += y[0];
            acc[i][j][r + 1] += y[1];
            acc[i][j][r + 2] += y[2];
            acc[i][j][r + 3] += y[3];
        });
    });
    static_assert(kF32DlPairFloats + 8 * 32 * 64 <= S * 2 * kF32DlOp, "epilogue staging must fit in the ring");
    float* stage = lds + kF32DlPairFloats + wave * 32 * 64;  // past the pair-reduction area
    if (!f32dl_store_fast<!A_KMAJ, !B_KMAJ>(p, acc, g, m0 + wm * 64, n0 + wn * 64, (int64_t)batch * p.stride_c,
                                            split, stage))
        store_wave<2, !A_KMAJ, !B_KMAJ>(p, acc, m0 + wm * 64, n0 + wn * 64, (int64_t)batch * p.stride_c, split, g);
}

// Small fp32 products (C1's layers, C4's fully connected layer): one block
// per 32 x 32 output tile and K chunk, so even a 64 x 256 x 784 product runs
// on ~200 blocks whose loads are all issued at once.  A block walks `cps`
// chunks of 64 k (the next chunk's loads in flight while the current one is
// summed from LDS) with plain FMAs: thread t owns column t % 32 and rows
// 4 (t / 32) .. +3 of the tile.  With more than one chunk group per tile,
// each block writes its partial tile and counts itself in on the tile's
// arrival counter; the block that arrives last adds the partials in chunk
// order (deterministic) and applies the epilogue, then resets the counter.
// The tile kernels above need a chain of load round trips per k block and a
// separate split-K reduction; at these sizes that latency, not arithmetic,
// set their 10-17 us per product.
constexpr int kSmT = 32;    // tile side
constexpr int kSmKC = 64;   // k per chunk
// One block of a small product: block `bid` of its grid (tile, chunk group).
template <bool A_KMAJ, bool B_KMAJ>
__device__ __forceinline__ void small_gemm_block(const GemmParams& p, int bid, int nchunks, int cps,
                                                 unsigned* __restrict__ tickets) {
    __shared__ float As[kSmKC][kSmT];   // As[k][m]
    __shared__ float Bs[kSmKC][kSmT];   // Bs[k][n]
    __shared__ int last;
    const int tile = bid / nchunks, chunk = bid - tile * nchunks;
    const int tm = tile / p.tiles_n, tn = tile - tm * p.tiles_n;
    const int m0 = tm * kSmT, n0 = tn * kSmT;
    const float* A = reinterpret_cast<const float*>(p.A);
    const float* B = reinterpret_cast<const float*>(p.B);
    const int t = threadIdx.x, col = t & 31, rg = t >> 5;

    // Loads of one 64-deep chunk: 512 float4 of A and 512 of B, two of each
    // per thread.  Element (m, k) of A is A[m*lda + k] (K-major) or
    // A[k*lda + m]; (k, n) of B is B[n*ldb + k] (K-major) or B[k*ldb + n].
    // A quad runs along the operand's contiguous dimension; out-of-range
    // elements read as zero.
    auto load_quad = [&](const float* X, int64_t ld, int mn0, int MN, bool kmaj, bool vec, int k0, int q) -> float4 {
        int mn, k;
        if (kmaj) { mn = q >> 4; k = k0 + 4 * (q & 15); }    // 32 rows x 16 quads along k
        else { k = k0 + (q >> 3); mn = 4 * (q & 7); }       // 64 k rows x 8 quads along m/n
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (kmaj) {
            const int row = mn0 + mn;
            if (row < MN) {
                const float* src = X + (int64_t)row * ld + k;
                if (vec && k + 4 <= p.K) {
                    const float4 w = *reinterpret_cast<const float4*>(src);
                    v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) if (k + e < p.K) v[e] = src[e];
                }
            }
        } else {
            if (k < p.K) {
                const int c0 = mn0 + mn;
                const float* src = X + (int64_t)k * ld + c0;
                if (vec && c0 + 4 <= MN) {
                    const float4 w = *reinterpret_cast<const float4*>(src);
                    v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) if (c0 + e < MN) v[e] = src[e];
                }
            }
        }
        return make_float4(v[0], v[1], v[2], v[3]);
    };
    auto store_quad = [&](float (*S)[kSmT], bool kmaj, int q, const float4& w) {
        if (kmaj) {
            const int mn = q >> 4, k = 4 * (q & 15);
            S[k][mn] = w.x; S[k + 1][mn] = w.y; S[k + 2][mn] = w.z; S[k + 3][mn] = w.w;
        } else {
            const int k = q >> 3, mn = 4 * (q & 7);
            *reinterpret_cast<float4*>(&S[k][mn]) = w;
        }
    };

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int kc_first = chunk * cps;
    const int kc_end = min(kc_first + cps, (p.K + kSmKC - 1) / kSmKC);
    float4 ra[2], rb[2];
    auto fetch = [&](int kc) {
        const int k0 = kc * kSmKC;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            ra[j] = load_quad(A, p.lda, m0, p.M, A_KMAJ, p.vec_a, k0, t + 256 * j);
            rb[j] = load_quad(B, p.ldb, n0, p.N, B_KMAJ, p.vec_b, k0, t + 256 * j);
        }
        if (p.mask_a) {
            // A ReLU's backward applied on the load: dy * (y > 0 ? 1 : 0),
            // the same product as the separate pass, so bit-identical.
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float4 y = load_quad(p.mask_a, p.lda, m0, p.M, A_KMAJ, p.vec_a, k0, t + 256 * j);
                ra[j].x *= y.x > 0.0f ? 1.0f : 0.0f;
                ra[j].y *= y.y > 0.0f ? 1.0f : 0.0f;
                ra[j].z *= y.z > 0.0f ? 1.0f : 0.0f;
                ra[j].w *= y.w > 0.0f ? 1.0f : 0.0f;
            }
        }
    };
    if (kc_first < kc_end) fetch(kc_first);
    for (int kc = kc_first; kc < kc_end; ++kc) {
        __syncthreads();   // the previous chunk's reads are done
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            store_quad(As, A_KMAJ, t + 256 * j, ra[j]);
            store_quad(Bs, B_KMAJ, t + 256 * j, rb[j]);
        }
        __syncthreads();
        if (kc + 1 < kc_end) fetch(kc + 1);
        const int kn = min(kSmKC, p.K - kc * kSmKC);
        for (int k = 0; k < kn; ++k) {
            const float4 a = *reinterpret_cast<const float4*>(&As[k][4 * rg]);
            const float b = Bs[k][col];
            acc[0] = fmaf(a.x, b, acc[0]);
            acc[1] = fmaf(a.y, b, acc[1]);
            acc[2] = fmaf(a.z, b, acc[2]);
            acc[3] = fmaf(a.w, b, acc[3]);
        }
    }

    if (nchunks > 1) {
        // Partials and counter go through agent-scope (cross-XCD coherent)
        // relaxed atomics, which need no cache maintenance; a block's stores
        // have completed (vmcnt 0 in every thread, then the barrier) before
        // it counts itself in.  A device-scope fence here instead writes
        // back and invalidates the XCD's L2 in every block: 208 blocks of a
        // 64 x 256 x 784 product took 35 us that way.
        float* part = p.partial + ((int64_t)tile * nchunks + chunk) * (kSmT * kSmT);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __hip_atomic_store(part + (4 * rg + i) * kSmT + col, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __syncthreads();
        if (t == 0)
            last = __hip_atomic_fetch_add(tickets + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (unsigned)(nchunks - 1);
        __syncthreads();
        if (!last) return;
        const float* base = p.partial + (int64_t)tile * nchunks * (kSmT * kSmT);
        auto ld = [&](int c, int i) {
            return __hip_atomic_load(base + (int64_t)c * (kSmT * kSmT) + (4 * rg + i) * kSmT + col, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        };
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = 0.0f;
        int c = 0;
        for (; c + 4 <= nchunks; c += 4) {
            float v[4][4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) v[u][i] = ld(c + u, i);
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] += v[u][i];
        }
        for (; c < nchunks; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += ld(c, i);
        if (t == 0) __hip_atomic_store(tickets + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    const int n = n0 + col;
    if (n >= p.N) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * rg + i;
        if (m >= p.M) break;
        const float bv = has_bias ? (p.row_bias ? p.bias[m] : p.bias[n]) : 0.0f;
        emit(p, (int64_t)m * p.ldc + n, acc[i], bv, relu);
    }
}

template <bool A_KMAJ, bool B_KMAJ>
__global__ __launch_bounds__(256) void gemm_f32_small_kernel(GemmParams p, int nchunks, int cps,
                                                             unsigned* __restrict__ tickets) {
    small_gemm_block<A_KMAJ, B_KMAJ>(p, blockIdx.x, nchunks, cps, tickets);
}

// Two small products in one launch (a Linear layer's dX = dY W and
// dW = dY^T X, which read the same dY): blocks [0, blocks1) are the first
// product's grid, the rest the second's, each block exactly as in its own
// launch (same tiles, chunk groups, order of sums), on separate arrival
// counters and partial buffers.
__global__ __launch_bounds__(256) void gemm_f32_small_pair_kernel(GemmParams p1, int nchunks1, int cps1,
                                                                  unsigned* __restrict__ tickets1, int blocks1,
                                                                  GemmParams p2, int nchunks2, int cps2,
                                                                  unsigned* __restrict__ tickets2) {
    if ((int)blockIdx.x < blocks1) small_gemm_block<true, false>(p1, blockIdx.x, nchunks1, cps1, tickets1);
    else small_gemm_block<false, false>(p2, blockIdx.x - blocks1, nchunks2, cps2, tickets2);
}

// Split-K reduction: C = epi(alpha * sum_s partial[s] + beta * C), summing the
// splits in ascending order (deterministic).  Grid (ceil(N / 1024), M): a
// block covers 1024 columns of one row, 4 per thread, with 16-byte loads of
// the partial rows when N % 4 == 0 (the workspace is 256-byte aligned).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmParams p, int splits) {
    const int col0 = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (col0 >= p.N) return;
    const int64_t plane = (int64_t)p.M * p.N;
    const int n = min(4, p.N - col0);
    const bool vec = n == 4 && (p.N & 3) == 0;
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    for (int row = blockIdx.y; row < p.M; row += gridDim.y) {
        const float* src = p.partial + (int64_t)row * p.N + col0;
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (vec) {
            // Eight splits' loads in flight at a time, added in split order.
            int k = 0;
            for (; k + 8 <= splits; k += 8) {
                float4 v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const float4*>(src + (k + u) * plane);
#pragma unroll
                for (int u = 0; u < 8; ++u) { s[0] += v[u].x; s[1] += v[u].y; s[2] += v[u].z; s[3] += v[u].w; }
            }
            if (k < splits) {
                float4 v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (k + u < splits) v[u] = *reinterpret_cast<const float4*>(src + (k + u) * plane);
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (k + u < splits) { s[0] += v[u].x; s[1] += v[u].y; s[2] += v[u].z; s[3] += v[u].w; }
            }
        } else {
            for (int k = 0; k < splits; ++k)
                for (int j = 0; j < n; ++j) s[j] += src[k * plane + j];
        }
        const float rb = (has_bias && p.row_bias) ? p.bias[row] : 0.0f;
        const int64_t off = (int64_t)row * p.ldc + col0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j >= n) break;
            float v = p.alpha * s[j];
            if (p.beta != 0.0f) v += p.beta * reinterpret_cast<const float*>(p.C)[off + j];
            if (has_bias) v += p.row_bias ? rb : p.bias[col0 + j];
            if (relu) v = fmaxf(v, 0.0f);
            if (p.out_bf16) reinterpret_cast<uint16_t*>(p.C)[off + j] = tfd::f32_to_bf16(v);
            else reinterpret_cast<float*>(p.C)[off + j] = v;
        }
    }
}

// Split-K reduction for many splits (>= 16) and small outputs: a block owns
// 16 consecutive output elements (flat index row * N + col) x 16 split
// groups; each thread adds splits g, g + 16, ... in ascending order with its
// loads in flight together, and the 16 group sums are combined in a fixed
// tree order before the epilogue (deterministic).
__global__ __launch_bounds__(256) void splitk_reduce_wide_kernel(GemmParams p, int splits) {
    __shared__ float red[16][17];
    const int el = threadIdx.x & 15, g = threadIdx.x >> 4;
    const int64_t plane = (int64_t)p.M * p.N;
    const int64_t i = (int64_t)blockIdx.x * 16 + el;
    float s = 0.0f;
    if (i < plane) {
#pragma unroll 8
        for (int k = g; k < splits; k += 16) s += p.partial[k * plane + i];
    }
    red[g][el] = s;
    __syncthreads();
    if (threadIdx.x >= 16 || i >= plane) return;
    float t[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) t[q] = red[2 * q][el] + red[2 * q + 1][el];
    const float sum = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
    const int row = (int)(i / p.N), col = (int)(i - (int64_t)row * p.N);
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    const int64_t off = (int64_t)row * p.ldc + col;
    float v = p.alpha * sum;
    if (p.beta != 0.0f) v += p.beta * reinterpret_cast<const float*>(p.C)[off];
    if (has_bias) v += p.row_bias ? p.bias[row] : p.bias[col];
    if (relu) v = fmaxf(v, 0.0f);
    if (p.out_bf16) reinterpret_cast<uint16_t*>(p.C)[off] = tfd::f32_to_bf16(v);
    else reinterpret_cast<float*>(p.C)[off] = v;
}

using KernelFn = void (*)(GemmParams);


// Narrow outputs over a long reduction, fp32: C = epi(alpha * A B^T) with
// A row-major [M x K] and B as [N x K] (trans_b), N <= 16 (a classifier
// forward: C4's 128 x 10 x 16384).  Block (c, g) takes the rows 8g .. 8g+7
// (a wave each) over the k chunk c of kSkC columns: the chunk of B (N x kSkC
// floats) is staged in LDS once per block, each lane multiplies 4
// consecutive k of its row, 256 apart, with all N rows of B, and a wave
// butterfly adds the N dot products.  With several chunks each row's N sums
// go to partials through agent-scope stores and the row group's last block
// (arrival counter) adds them in chunk order (deterministic), then applies
// alpha, the bias and ReLU.  C4's shape: 12.7 us, where the tiled kernel and
// its split-K reduction took 12.9 + 4.4 us; what remains is the chain of
// latencies (loads, partial stores, the counter, the last block's loads).
constexpr int kSkN = 16, kSkC = 1024, kSkRows = 8;
__global__ __launch_bounds__(512) void gemm_f32_skinny_kernel(GemmParams p, int chunks, unsigned* __restrict__ tickets) {
    __shared__ float4 bs[kSkN][kSkC / 4];
    __shared__ bool last;
    const int N = p.N, K = p.K, M = p.M;
    const int c = blockIdx.x, g = blockIdx.y;
    const int k0 = c * kSkC;
    const float* A = reinterpret_cast<const float*>(p.A);
    const float* B = reinterpret_cast<const float*>(p.B);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m = g * kSkRows + wave;
    // This lane's A values first, so their latency overlaps the B staging.
    float4 av[kSkC / 256];
#pragma unroll
    for (int j = 0; j < kSkC / 256; ++j) {
        const int k = k0 + 4 * (lane + 64 * j);
        const float* a = A + (int64_t)min(m, M - 1) * p.lda;
        if (p.vec_a && k + 4 <= K) {
            av[j] = *reinterpret_cast<const float4*>(a + k);
        } else {
            av[j].x = k + 0 < K ? a[k + 0] : 0.0f;
            av[j].y = k + 1 < K ? a[k + 1] : 0.0f;
            av[j].z = k + 2 < K ? a[k + 2] : 0.0f;
            av[j].w = k + 3 < K ? a[k + 3] : 0.0f;
        }
    }
    // The B chunk: all of this thread's loads in flight, then the LDS stores.
    constexpr int kSkPer = kSkN * (kSkC / 4) / 512;
    float4 bv[kSkPer];
#pragma unroll
    for (int r = 0; r < kSkPer; ++r) {
        const int i = threadIdx.x + 512 * r;
        const int n = i / (kSkC / 4), q = i % (kSkC / 4), k = k0 + 4 * q;
        bv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (n < N) {
            const float* src = B + (int64_t)n * p.ldb + k;
            if (p.vec_b && k + 4 <= K) {
                bv[r] = *reinterpret_cast<const float4*>(src);
            } else {
                bv[r].x = k + 0 < K ? src[0] : 0.0f;
                bv[r].y = k + 1 < K ? src[1] : 0.0f;
                bv[r].z = k + 2 < K ? src[2] : 0.0f;
                bv[r].w = k + 3 < K ? src[3] : 0.0f;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kSkPer; ++r) {
        const int i = threadIdx.x + 512 * r;
        bs[i / (kSkC / 4)][i % (kSkC / 4)] = bv[r];
    }
    __syncthreads();
    float acc[kSkN];
#pragma unroll
    for (int n = 0; n < kSkN; ++n) acc[n] = 0.0f;
    if (m < M) {
#pragma unroll
        for (int j = 0; j < kSkC / 256; ++j)
#pragma unroll
            for (int n = 0; n < kSkN; ++n) {
                if (n >= N) break;
                const float4 b = bs[n][lane + 64 * j];
                acc[n] += av[j].x * b.x + av[j].y * b.y + av[j].z * b.z + av[j].w * b.w;
            }
    }
#pragma unroll
    for (int n = 0; n < kSkN; ++n)
        if (n < N) acc[n] = tfd::wave_sum(acc[n]);
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    auto finish = [&](int row, int n, float sum) {
        float v = p.alpha * sum;
        if (has_bias) v += p.row_bias ? p.bias[row] : p.bias[n];
        if (relu) v = fmaxf(v, 0.0f);
        reinterpret_cast<float*>(p.C)[(int64_t)row * p.ldc + n] = v;
    };
    // Lane n holds the row's n-th sum (every lane holds all of them after
    // the butterfly; lane n keeps acc[n]).
    float mine = 0.0f;
#pragma unroll
    for (int n = 0; n < kSkN; ++n)
        if (lane == n) mine = acc[n];
    if (chunks == 1) {
        if (m < M && lane < N) finish(m, lane, mine);
        return;
    }
    if (m < M && lane < N)
        __hip_atomic_store(p.partial + ((int64_t)c * M + m) * N + lane, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    tfd::wait_stores_landed();   // the partials have landed
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(tickets + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(chunks - 1);
    __syncthreads();
    if (!last) return;
    if (m < M && lane < N) {
        const float* sp = p.partial + (int64_t)m * N + lane;
        const int64_t step = (int64_t)M * N;
        float v = 0.0f;
        int k = 0;
        for (; k + 8 <= chunks; k += 8) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = __hip_atomic_load(sp + (k + u) * step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int u = 0; u < 8; ++u) v += t[u];
        }
        for (; k < chunks; ++k) v += __hip_atomic_load(sp + k * step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        finish(m, lane, v);
    }
    if (threadIdx.x == 0) __hip_atomic_store(tickets + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Narrow fp32 outputs (N <= 16) over a long K on MFMA: 16 rows x 512 k per
// block, v_mfma_f32_16x16x4f32 with A[i][k] = row i of A and B[k][j] = row j
// of B (as [N x K]).  Lane (i = l % 16, q = l / 16) loads A[row i][k .. k+3]
// and B[row i][k .. k+3] with k = base + 16 j + 4 q, and feeds element s to
// the s-th of four MFMAs, so each k of the wave's 64 enters once and the
// lanes' partial dot products are summed by the MFMA itself (no butterflies,
// no staging).  The eight waves' 16 x 16 tiles are added in order through
// LDS; with several k chunks each block stores its 16 x N partial and the
// row group's last block adds the chunks in order (as gemm_f32_skinny_kernel,
// which serves operands that are not 16-byte loadable).
constexpr int kNmRows = 16, kNmKC = 512;
__global__ __launch_bounds__(512) void gemm_f32_narrow_mfma_kernel(GemmParams p, int chunks,
                                                                   unsigned* __restrict__ tickets) {
    __shared__ float red[8][kNmRows][17];
    __shared__ bool last;
    const int M = p.M, N = p.N, K = p.K;
    const int c = blockIdx.x, g = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, q = lane >> 4;
    const int row = g * kNmRows + l16;
    const int kw0 = c * kNmKC + wave * (kNmKC / 8);
    const float* A = reinterpret_cast<const float*>(p.A) + (int64_t)min(row, M - 1) * p.lda;
    const float* B = reinterpret_cast<const float*>(p.B) + (int64_t)min(l16, N - 1) * p.ldb;
    float4 av[4], bv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = kw0 + 16 * j + 4 * q;   // K % 4 == 0: the quad is wholly in or out
        av[j] = row < M && k < K ? *reinterpret_cast<const float4*>(A + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        bv[j] = l16 < N && k < K ? *reinterpret_cast<const float4*>(B + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].x, bv[j].x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].y, bv[j].y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].z, bv[j].z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].w, bv[j].w, acc, 0, 0, 0);
    }
    // acc[r] = D[4 q + r][l16]: row 4 q + r of the group, output column l16.
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * q + r][l16] = acc[r];
    __syncthreads();
    const int t = threadIdx.x, i = t >> 4, j = t & 15;   // threads 0 .. 255: (row i, column j)
    const int orow = g * kNmRows + i;
    const bool mine = t < kNmRows * 16 && orow < M && j < N;
    float v = 0.0f;
    if (mine) {
#pragma unroll
        for (int w = 0; w < 8; ++w) v += red[w][i][j];
    }
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    auto finish = [&](float sum) {
        float o = p.alpha * sum;
        if (has_bias) o += p.row_bias ? p.bias[orow] : p.bias[j];
        if (relu) o = fmaxf(o, 0.0f);
        reinterpret_cast<float*>(p.C)[(int64_t)orow * p.ldc + j] = o;
    };
    if (chunks == 1) {
        if (mine) finish(v);
        return;
    }
    if (mine) __hip_atomic_store(p.partial + ((int64_t)c * M + orow) * N + j, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    tfd::wait_stores_landed();   // the partials have landed
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(tickets + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(chunks - 1);
    __syncthreads();
    if (!last) return;
    if (mine) {
        // The chunks' partials in chunk order, 32 loads in flight (clamped
        // addresses; the ones past the last chunk are not added).
        const float* sp = p.partial + (int64_t)orow * N + j;
        const int64_t step = (int64_t)M * N;
        float s = 0.0f;
        for (int k = 0; k < chunks; k += 32) {
            float t32[32];
#pragma unroll
            for (int u = 0; u < 32; ++u)
                t32[u] = __hip_atomic_load(sp + min(k + u, chunks - 1) * step, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int u = 0; u < 32; ++u)
                if (k + u < chunks) s += t32[u];
        }
        finish(s);
    }
    if (threadIdx.x == 0) __hip_atomic_store(tickets + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// fp32 GEMM with a short K (<= 32) and few rows (<= 64), A K-major and B
// MN-major: a convolution over few input channels (W [Cout x Cin*k*k] times
// each image's im2col block).  An MFMA tile would be mostly padding and one
// latency-bound k block, so one VALU thread per output column n (of one
// batch element) keeps its K values of B in registers and produces all M
// rows.  A sits in LDS zero-padded to 32 columns (the reads are uniform, so
// they broadcast), which makes every row 32 unconditional FMAs, and the B
// loads are unconditional too (rows past K re-read row K-1 and are then
// replaced by zeros).  Sums run over k ascending.
__global__ __launch_bounds__(256) void gemm_f32_smallk_kernel(GemmParams p) {
    __shared__ float As[64 * 32];
    const int64_t b = blockIdx.y;
    const float* A = reinterpret_cast<const float*>(p.A) + b * p.stride_a;
    for (int i = threadIdx.x; i < 64 * 32; i += 256) {
        const int m = i >> 5, k = i & 31;
        As[i] = (m < p.M && k < p.K) ? A[(int64_t)m * p.lda + k] : 0.0f;
    }
    __syncthreads();
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= p.N) return;
    float bk[32];
    if (p.K > 0) {
        const float* B = reinterpret_cast<const float*>(p.B) + b * p.stride_b + n;
        const int klast = p.K - 1;
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const float v = B[(int64_t)min(k, klast) * p.ldb];
            bk[k] = k <= klast ? v : 0.0f;  // a select, not a branch: an inf in row K-1 must not meet a 0
        }
    } else {
#pragma unroll
        for (int k = 0; k < 32; ++k) bk[k] = 0.0f;
    }
    const bool has_bias = p.epi != TF_EPI_NONE && p.epi != TF_EPI_RELU;
    const bool relu = p.epi == TF_EPI_BIAS_RELU || p.epi == TF_EPI_RELU || p.epi == TF_EPI_ROW_BIAS_RELU;
    const float col_bias = (has_bias && !p.row_bias) ? p.bias[n] : 0.0f;
    const int64_t c0 = b * p.stride_c + n;
    for (int m = 0; m < p.M; ++m) {
        const float* a = As + m * 32;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 32; ++k) acc = fmaf(a[k], bk[k], acc);
        emit(p, c0 + (int64_t)m * p.ldc, acc, has_bias ? (p.row_bias ? p.bias[m] : col_bias) : 0.0f, relu);
    }
}

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

KernelFn pick_f32_dl(bool a_kmaj, bool b_kmaj) {
    if (a_kmaj && b_kmaj) return gemm_f32_dl_kernel<true, true>;
    if (a_kmaj && !b_kmaj) return gemm_f32_dl_kernel<true, false>;
    if (!a_kmaj && b_kmaj) return gemm_f32_dl_kernel<false, true>;
    return gemm_f32_dl_kernel<false, false>;
}

KernelFn pick_bf16_big(bool a_kmaj, bool b_kmaj) {
    if (a_kmaj && b_kmaj) return gemm_bf16_big_kernel<true, true>;
    if (a_kmaj && !b_kmaj) return gemm_bf16_big_kernel<true, false>;
    if (!a_kmaj && b_kmaj) return gemm_bf16_big_kernel<false, true>;
    return gemm_bf16_big_kernel<false, false>;
}

// Interior bf16 tiles run on the eight-wave ping-pong kernel (2-3 % faster
// than the eight-wave kernel on the C5 backward GEMMs, which itself was
// 3.5-5 % faster than four waves).  Building with -DTF_BF16_KERNEL=1 selects
// the eight-wave kernel, 0 the four-wave one.  (The eight-wave kernel for the
// weight-gradient layout alone, both operands MN-major, was measured 0.4 %
// slower on the config-5 step, though faster on N(0,1) operands.)
#ifndef TF_BF16_KERNEL
#define TF_BF16_KERNEL 2
#endif
constexpr int kBf16Kernel = TF_BF16_KERNEL;
constexpr int kBf16DlThreads = kBf16Kernel >= 1 ? 2 * kThreads : kThreads;
KernelFn pick_bf16_dl(bool a_kmaj, bool b_kmaj, bool ktail) {
    if constexpr (kBf16Kernel == 2) {
        if (ktail) {
            if (a_kmaj && b_kmaj) return gemm_bf16_pp_kernel<true, true, true>;
            if (a_kmaj && !b_kmaj) return gemm_bf16_pp_kernel<true, false, true>;
            if (!a_kmaj && b_kmaj) return gemm_bf16_pp_kernel<false, true, true>;
            return gemm_bf16_pp_kernel<false, false, true>;
        }
        if (a_kmaj && b_kmaj) return gemm_bf16_pp_kernel<true, true, false>;
        if (a_kmaj && !b_kmaj) return gemm_bf16_pp_kernel<true, false, false>;
        if (!a_kmaj && b_kmaj) return gemm_bf16_pp_kernel<false, true, false>;
        return gemm_bf16_pp_kernel<false, false, false>;
    } else if constexpr (kBf16Kernel == 1) {
        if (ktail) {
            if (a_kmaj && b_kmaj) return gemm_bf16_dl8_kernel<true, true, true>;
            if (a_kmaj && !b_kmaj) return gemm_bf16_dl8_kernel<true, false, true>;
            if (!a_kmaj && b_kmaj) return gemm_bf16_dl8_kernel<false, true, true>;
            return gemm_bf16_dl8_kernel<false, false, true>;
        }
        if (a_kmaj && b_kmaj) return gemm_bf16_dl8_kernel<true, true>;
        if (a_kmaj && !b_kmaj) return gemm_bf16_dl8_kernel<true, false>;
        if (!a_kmaj && b_kmaj) return gemm_bf16_dl8_kernel<false, true>;
        return gemm_bf16_dl8_kernel<false, false>;
    } else {
        if (a_kmaj && b_kmaj) return gemm_bf16_dl_kernel<true, true>;
        if (a_kmaj && !b_kmaj) return gemm_bf16_dl_kernel<true, false>;
        if (!a_kmaj && b_kmaj) return gemm_bf16_dl_kernel<false, true>;
        return gemm_bf16_dl_kernel<false, false>;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Split count for a grid of `tiles` workgroups over `kblocks` k blocks:
// enough slices for `target` workgroups, each slice >= min_per k blocks.
int choose_splits(int64_t tiles, int64_t kblocks, int64_t target, int64_t min_per) {
    if (tiles >= target || kblocks < 2 * min_per) return 1;
    const int64_t want = (target + tiles - 1) / tiles;
    return (int)std::max<int64_t>(1, std::min<int64_t>({want, kblocks / min_per, 256}));
}

// Split-K partials of tf_gemm_noalloc: a fixed device array instead of the
// context's pool-grown workspace.  64 MiB covers every split this library
// chooses for the benchmark configurations (the largest, config 5's
// 4096 x 1000 products over 4 K slices, needs 65.5 MB); a split that needs
// more is rejected.  Each GPU the library runs on holds its own copy until
// the process ends.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// Device address of `scratch` on `device`, looked up once per device with
// that device current.  The array's name is only a host-side stand-in.
tf_status scratch_address(int device, float** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    TF_REQUIRE(device >= 0 && device < kMaxDevices, "tf_gemm_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (addr[device] == nullptr) {
        int cur = -1;
        TF_HIP_CHECK(hipGetDevice(&cur));
        if (cur != device) TF_HIP_CHECK(hipSetDevice(device));
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != device) (void)hipSetDevice(cur);
        if (e != hipSuccess) return tfh::hip_error(e, "tf_gemm_noalloc: hipGetSymbolAddress(scratch)");
        TF_REQUIRE(p != nullptr, "tf_gemm_noalloc: null scratch address");
        addr[device] = p;
    }
    *out = static_cast<float*>(addr[device]);
    return TF_OK;
}

// Where a launch's cross-block partials go: the fixed scratch array for
// tf_gemm_noalloc (rejected, with one message for every kernel path, when
// they need more than it holds), else the context's pool-grown workspace.
tf_status partials_buffer(tf_ctx* ctx, size_t need, bool noalloc, float** out) {
    if (noalloc) {
        if (need > kNoAllocScratchBytes)
            return tfh::set_error(TF_ERR_INVALID,
                                  "tf_gemm_noalloc: this shape's partial sums need " + std::to_string(need) +
                                      " bytes, more than the fixed scratch of " +
                                      std::to_string(kNoAllocScratchBytes) + " bytes (use tf_gemm)");
        return scratch_address(ctx->device, out);
    }
    tf_status st = tfh::ensure_workspace(ctx, need);
    if (st != TF_OK) return st;
    *out = reinterpret_cast<float*>(ctx->ws);
    return TF_OK;
}

// Grid of the small-product kernel for an M x N x K product: 32 x 32 tiles
// and enough chunk groups for ~256 blocks, at most 32 per tile (the last
// block adds them up), each of >= 1 chunk of 64 k.  False when the product
// does not fit that kernel.
bool small_grid(int64_t ncu, int64_t M, int64_t N, int64_t K, int64_t& tiles, int64_t& groups, int& cps) {
    tiles = ((M + kSmT - 1) / kSmT) * ((N + kSmT - 1) / kSmT);
    if (!(K > 0 && K <= 2048 && (double)M * (double)N * (double)K <= 134217728.0 && tiles <= tfh::kTicketGemmTiles))
        return false;
    const int64_t nkc = (K + kSmKC - 1) / kSmKC;
    groups = std::min<int64_t>({nkc, 32, std::max<int64_t>(1, (ncu + tiles - 1) / tiles)});
    cps = (int)((nkc + groups - 1) / groups);
    groups = (nkc + cps - 1) / cps;
    return true;
}

// `noalloc`: split-K partials go to the fixed scratch array (no pool call).
tf_status gemm_impl(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                    const void* A, int64_t lda, int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b,
                    float beta, void* C, int64_t ldc, int64_t stride_c, int64_t batch, int reduce_batch,
                    int in_dtype, int out_dtype, int epi, const float* bias, bool noalloc = false,
                    const float* mask_a = nullptr) {
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
    TF_REQUIRE(!mask_a || (in_dtype == TF_F32 && batch == 1 && !reduce_batch), "tf_gemm: a mask needs one Float32 product");

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
    const int64_t ncu = ctx->num_cus;
    // bf16 with enough work for one 256 x 256 tile per CU (directly, or with
    // K split over at most 4 slices of >= 8 k blocks): the large-tile kernel.
    bool big = false;
    int splits = 1;
    if (in_dtype == TF_BF16 && M >= 128 && N >= 128) {
        const int64_t tb = ((M + kBigTile - 1) / kBigTile) * ((N + kBigTile - 1) / kBigTile) * grid_batch;
        const int64_t kb = ((K + kBigK - 1) / kBigK) * (reduce_batch ? batch : 1);
        const int s = grid_batch == 1 ? choose_splits(tb, kb, ncu, 8) : 1;
        if (tb * s >= ncu && s <= 4) {
            big = true;
            splits = s;
        }
    }
    // Otherwise: tile width 128 x 128 when that gives every CU at least its
    // resident workgroup count (fp32: one, its three LDS stages take 108 KB;
    // bf16: two, which hide each other's barrier and LDS latency), 128 x 64
    // otherwise and for narrow outputs.
    const int64_t per_cu = in_dtype == TF_F32 ? 1 : 2;
    const int64_t tiles_m = big ? (M + kBigTile - 1) / kBigTile : (M + BM - 1) / BM;
    const int64_t t128 = tiles_m * ((N + 127) / 128) * grid_batch;
    const int BN = big ? kBigTile : (N <= 64 || t128 < per_cu * ncu) ? 64 : 128;
    p.tiles_m = (int)tiles_m;
    p.tiles_n = (int)((N + BN - 1) / BN);
    p.alpha = alpha; p.beta = beta; p.epi = epi; p.row_bias = row_bias;
    p.out_bf16 = out_dtype == TF_BF16;
    p.reduce_batch = reduce_batch ? (int)batch : 1;
    p.vec_a = aligned16(A) && (lda % vec_elems == 0) && (stride_a % vec_elems == 0);
    p.vec_b = aligned16(B) && (ldb % vec_elems == 0) && (stride_b % vec_elems == 0);
    p.mask_a = mask_a;
    if (mask_a && !aligned16(mask_a)) p.vec_a = 0;
    p.pair_c = (reinterpret_cast<uintptr_t>(C) & 7) == 0 && (ldc % 2 == 0) && (p.stride_c % 2 == 0);
    const uintptr_t c_vec_bytes = out_dtype == TF_BF16 ? 8 : 16;
    p.vec_c4 = (reinterpret_cast<uintptr_t>(C) & (c_vec_bytes - 1)) == 0 && (ldc % 4 == 0) && (p.stride_c % 4 == 0);
    // Narrow fp32 outputs (K >= 64), 16-byte loadable operands: the MFMA form
    // (gemm_f32_narrow_mfma_kernel; one k chunk, no partials, below 513).
    if (!mask_a && in_dtype == TF_F32 && out_dtype == TF_F32 && batch == 1 && !reduce_batch && a_kmaj && b_kmaj && N <= 16 &&
        K >= 64 && K % 4 == 0 && p.vec_a && p.vec_b && beta == 0.0f &&
        (M + kNmRows - 1) / kNmRows <= tfh::kTicketGemmTiles) {
        const int64_t chunks = (K + kNmKC - 1) / kNmKC;
        const int64_t groups = (M + kNmRows - 1) / kNmRows;
        TF_REQUIRE(chunks < 65536 && groups < 65536, "tf_gemm: narrow grid too large");
        if (chunks > 1) {
            const size_t need = (size_t)chunks * (size_t)M * (size_t)N * sizeof(float);
            tf_status st = partials_buffer(ctx, need, noalloc, &p.partial);
            if (st != TF_OK) return st;
        }
        gemm_f32_narrow_mfma_kernel<<<dim3((unsigned)chunks, (unsigned)groups), 512, 0, ctx->stream>>>(
            p, (int)chunks, ctx->tickets + tfh::kTicketGemm);
        return tfh::check_launch("gemm_f32_narrow_mfma_kernel");
    }
    // Narrow fp32 outputs over a long K (see gemm_f32_skinny_kernel).
    if (!mask_a && in_dtype == TF_F32 && out_dtype == TF_F32 && batch == 1 && !reduce_batch && a_kmaj && b_kmaj && N <= kSkN &&
        K >= 2048 && beta == 0.0f && (M + kSkRows - 1) / kSkRows <= tfh::kTicketGemmTiles) {
        const int64_t chunks = (K + kSkC - 1) / kSkC;
        const int64_t groups = (M + kSkRows - 1) / kSkRows;
        TF_REQUIRE(chunks < 65536 && groups < 65536, "tf_gemm: skinny grid too large");
        if (chunks > 1) {
            const size_t need = (size_t)chunks * (size_t)M * (size_t)N * sizeof(float);
            tf_status st = partials_buffer(ctx, need, noalloc, &p.partial);
            if (st != TF_OK) return st;
        }
        gemm_f32_skinny_kernel<<<dim3((unsigned)chunks, (unsigned)groups), 512, 0, ctx->stream>>>(
            p, (int)chunks, ctx->tickets + tfh::kTicketGemm);
        return tfh::check_launch("gemm_f32_skinny_kernel");
    }
    // Small fp32 products: 32 x 32 tiles with K over many blocks (see
    // gemm_f32_small_kernel).
    int64_t sm_tiles = 0, groups = 0;
    int cps = 0;
    if (in_dtype == TF_F32 && batch == 1 && small_grid(ncu, M, N, K, sm_tiles, groups, cps)) {
        p.tiles_m = (int)((M + kSmT - 1) / kSmT);
        p.tiles_n = (int)((N + kSmT - 1) / kSmT);
        if (groups > 1) {
            const size_t need = (size_t)sm_tiles * (size_t)groups * kSmT * kSmT * sizeof(float);
            tf_status st = partials_buffer(ctx, need, noalloc, &p.partial);
            if (st != TF_OK) return st;
        }
        const dim3 grid((unsigned)(sm_tiles * groups));
        unsigned* tickets = ctx->tickets + tfh::kTicketGemm;
        if (a_kmaj && b_kmaj) gemm_f32_small_kernel<true, true><<<grid, 256, 0, ctx->stream>>>(p, (int)groups, cps, tickets);
        else if (a_kmaj) gemm_f32_small_kernel<true, false><<<grid, 256, 0, ctx->stream>>>(p, (int)groups, cps, tickets);
        else if (b_kmaj) gemm_f32_small_kernel<false, true><<<grid, 256, 0, ctx->stream>>>(p, (int)groups, cps, tickets);
        else gemm_f32_small_kernel<false, false><<<grid, 256, 0, ctx->stream>>>(p, (int)groups, cps, tickets);
        return tfh::check_launch("gemm_f32_small_kernel");
    }
    if (mask_a)
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_gemm_relu_masked: the masked operand needs a Float32 product with "
                                                  "K <= 2048 and M*N*K <= 2^27 (the small-product kernel)");
    if (in_dtype == TF_F32 && !trans_a && !trans_b && !reduce_batch && K <= 32 && M <= 64 && N >= 256) {
        const dim3 grid((unsigned)((N + 255) / 256), (unsigned)batch);
        gemm_f32_smallk_kernel<<<grid, 256, 0, ctx->stream>>>(p);
        return tfh::check_launch("gemm_f32_smallk_kernel");
    }
    if (big) {
        // Interior tiles take the direct-to-LDS kernel when the operands are
        // 16-byte loadable, K is a whole number of 16-byte loads (both
        // kernels count splits in 64-deep blocks, the last one partial when
        // K % 64 != 0, so their split boundaries agree) and each operand's
        // extent fits the buffer descriptor.
        const int64_t ext_a = trans_a ? (K - 1) * lda + M : (M - 1) * lda + K;
        const int64_t ext_b = trans_b ? (N - 1) * ldb + K : (K - 1) * ldb + N;
        const int64_t lim = (int64_t)0x7fffffff;  // descriptor extent is passed as int
        const int64_t k_unit = kBf16Kernel >= 1 ? 8 : 64;   // the four-wave kernel has no K tail
        const bool direct = K > 0 && K % k_unit == 0 && p.vec_a && p.vec_b && ext_a * esz <= lim && ext_b * esz <= lim;
        p.a_bytes = direct ? (uint32_t)(ext_a * esz) : 0u;
        p.b_bytes = direct ? (uint32_t)(ext_b * esz) : 0u;
        // Partial tiles at the M / N edges are fine for the direct kernel:
        // rows past an operand's extent read as zero (buffer range check),
        // rows past M or N inside it only feed outputs that are not stored.
        // An MN-major operand needs its row count a multiple of 8 for that,
        // so no 16-byte load straddles the end of its extent.
        const bool part_m = trans_a == 0 || M % 8 == 0;
        const bool part_n = trans_b != 0 || N % 8 == 0;
        p.int_m = direct ? (int)(part_m ? (M + kBigTile - 1) / kBigTile : M / kBigTile) : 0;
        p.int_n = direct ? (int)(part_n ? (N + kBigTile - 1) / kBigTile : N / kBigTile) : 0;
    }

    // fp32 with 128 x 128 tiles: the tiles of an int_m x int_n grid take the
    // direct-to-LDS kernel when K is a whole number of 32-deep blocks, the
    // operands are 16-byte loadable and each extent fits the descriptor.
    // Partial tiles at the M / N edges are fine for it as for the bf16 one;
    // an MN-major operand needs its row count a multiple of 4 for that.
    bool dl32 = false;
    if (in_dtype == TF_F32 && BN == 128) {
        const int64_t ext_a = trans_a ? (K - 1) * lda + M : (M - 1) * lda + K;
        const int64_t ext_b = trans_b ? (N - 1) * ldb + K : (K - 1) * ldb + N;
        const int64_t lim = (int64_t)0x7fffffff;
        if (K > 0 && K % 32 == 0 && p.vec_a && p.vec_b && ext_a * 4 <= lim && ext_b * 4 <= lim) {
            const bool part_m = trans_a == 0 || M % 4 == 0;
            const bool part_n = trans_b != 0 || N % 4 == 0;
            p.int_m = part_m ? p.tiles_m : (int)(M / BM);
            p.int_n = part_n ? p.tiles_n : (int)(N / 128);
            p.a_bytes = (uint32_t)(ext_a * 4);
            p.b_bytes = (uint32_t)(ext_b * 4);
            dl32 = p.int_m * p.int_n > 0;
            if (!dl32) p.int_m = p.int_n = 0;
        }
    }

    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    TF_REQUIRE(tiles < (1LL << 31), "tf_gemm: too many tiles");

    // Split the k blocks when the tiles leave most CUs idle and K is long
    // (target: the resident workgroups of every CU, >= 4 k blocks per slice).
    const int64_t kblocks = ((K + BK - 1) / BK) * p.reduce_batch;
    if (!big && grid_batch == 1 && tiles * 2 <= ncu && kblocks >= 8)
        splits = choose_splits(tiles, kblocks, per_cu * ncu, 4);
    if (kblocks == 0) {
        splits = 1;
        p.kb_per_split = 0;
    } else {
        int64_t per = (kblocks + splits - 1) / splits;
        splits = (int)((kblocks + per - 1) / per);
        p.kb_per_split = (int)per;
    }

    if (splits > 1) {
        const size_t need = (size_t)splits * (size_t)M * (size_t)N * sizeof(float);
        tf_status st = partials_buffer(ctx, need, noalloc, &p.partial);
        if (st != TF_OK) return st;
    }

    tf_status st = TF_OK;
    if (big) {
        // Direct-to-LDS kernel over an int_m x int_n grid of tiles; the
        // remaining edge tiles (or all tiles): the guarded kernel.
        const int64_t n_int = (int64_t)p.int_m * p.int_n;
        if (n_int > 0) {
            GemmParams q = p;
            q.tiles_m = p.int_m;
            q.tiles_n = p.int_n;
            dim3 grid((unsigned)n_int, (unsigned)splits, (unsigned)grid_batch);
            pick_bf16_dl(a_kmaj, b_kmaj, K % 64 != 0)<<<grid, kBf16DlThreads, 0, ctx->stream>>>(q);
            st = tfh::check_launch("gemm_bf16_dl_kernel");
            if (st != TF_OK) return st;
        }
        if (tiles - n_int > 0) {
            dim3 grid((unsigned)(tiles - n_int), (unsigned)splits, (unsigned)grid_batch);
            pick_bf16_big(a_kmaj, b_kmaj)<<<grid, kThreads, 0, ctx->stream>>>(p);
            st = tfh::check_launch("gemm_bf16_big_kernel");
            if (st != TF_OK) return st;
        }
    } else if (dl32) {
        const int64_t n_int = (int64_t)p.int_m * p.int_n;
        GemmParams q = p;
        q.tiles_m = p.int_m;
        q.tiles_n = p.int_n;
        dim3 grid((unsigned)n_int, (unsigned)splits, (unsigned)grid_batch);
        pick_f32_dl(a_kmaj, b_kmaj)<<<grid, kF32DlThreads, 0, ctx->stream>>>(q);
        st = tfh::check_launch("gemm_f32_dl_kernel");
        if (st != TF_OK) return st;
        if (tiles - n_int > 0) {
            dim3 egrid((unsigned)(tiles - n_int), (unsigned)splits, (unsigned)grid_batch);
            pick_f32<128>(a_kmaj, b_kmaj)<<<egrid, kThreads, 0, ctx->stream>>>(p);
            st = tfh::check_launch("gemm_f32_kernel");
            if (st != TF_OK) return st;
        }
    } else {
        KernelFn fn = in_dtype == TF_F32 ? (BN == 128 ? pick_f32<128>(a_kmaj, b_kmaj) : pick_f32<64>(a_kmaj, b_kmaj))
                                         : (BN == 128 ? pick_bf16<128>(a_kmaj, b_kmaj) : pick_bf16<64>(a_kmaj, b_kmaj));
        dim3 grid((unsigned)tiles, (unsigned)splits, (unsigned)grid_batch);
        fn<<<grid, kThreads, 0, ctx->stream>>>(p);
        st = tfh::check_launch("gemm kernel");
        if (st != TF_OK) return st;
    }
    if (splits > 1) {
        if (splits >= 16) {
            splitk_reduce_wide_kernel<<<(unsigned)((M * N + 15) / 16), 256, 0, ctx->stream>>>(p, splits);
        } else {
            dim3 rgrid((unsigned)((N + 1023) / 1024), (unsigned)std::min<int64_t>(M, 65535));
            splitk_reduce_kernel<<<rgrid, 256, 0, ctx->stream>>>(p, splits);
        }
        st = tfh::check_launch("splitk_reduce_kernel");
    }
    return st;
}


// ---------------------------------------------------------------------------
// Backward of a Linear layer with few outputs (N <= 16, fp32), in one launch:
//   dX[r][k] = sum_n dY[r][n] W[n][k],  dW[n][k] = sum_r dY[r][n] X[r][k],
//   db[n] = sum_r dY[r][n]
// (nn/Linear.cpp's backward as LinearBackward forms it: two GEMMs and a
// column sum).  Block b owns columns 64 b .. 64 b + 63 of K for every row, so
// dW needs no sum across blocks: thread t takes the column quad t % 16 of
// rows t / 16, t / 16 + 16, ... (a batch of eight rows' X loads in flight),
// adds its rows in ascending order, and the 16 row groups are added in order
// through LDS.  dY goes through LDS a batch of 128 rows at a time (as laid
// out in memory, read back as NP values a row, N rounded up to 4, zero past
// N), and the block's 64 columns of W sit in registers, so the loops over n
// have no branches and no load waits inside them.  All of a batch's loads
// (dY, X, and W in the first batch) are in flight together.  Block 0 also
// sums db (each row group's rows in order, then the 16 groups in order).
// Deterministic; every output written once.
// ---------------------------------------------------------------------------
constexpr int kLnbCols = 64, kLnbMaxN = 16, kLnbRows = 8, kLnbBatch = 16 * kLnbRows;
template <int NP, bool DVEC>
__global__ __launch_bounds__(256) void linear_bwd_narrow_kernel(const float* __restrict__ dy,
                                                                const float* __restrict__ x,
                                                                const float* __restrict__ w, float* __restrict__ dx,
                                                                float* __restrict__ dw, float* __restrict__ db, int M,
                                                                int N, int K) {
    static_assert(NP % 4 == 0 && NP <= kLnbMaxN, "NP: N rounded up to 4, at most 16");
    __shared__ float4 dys[kLnbBatch * kLnbMaxN / 4];    // one batch of dY rows, as in memory (N a row)
    extern __shared__ float red[];                       // [16][N][64]
    const float* dyf = reinterpret_cast<const float*>(dys);
    const int t = threadIdx.x, cq = t & 15, rg = t >> 4;
    const int k0 = blockIdx.x * kLnbCols, kq = k0 + 4 * cq;
    const bool colok = kq < K;                           // K % 4 == 0: a quad is wholly in or out
    const int kc = colok ? kq : 0;
    // X rows come from x when dW is wanted, else (values unused) from row 0
    // of w, so the loads need no branch around them.
    const float* xb = dw ? x : w;
    const int64_t xld = dw ? K : 0;
    float4 acc[NP];
#pragma unroll
    for (int n = 0; n < NP; ++n) acc[n] = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 wv[NP];
#pragma unroll
    for (int n = 0; n < NP; ++n) {
        const float4 v = *reinterpret_cast<const float4*>(w + (int64_t)min(n, N - 1) * K + kc);
        wv[n] = n < N && colok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float dbv = 0.0f;
    for (int rb0 = 0; rb0 < M; rb0 += kLnbBatch) {
        // The batch's dY, then its X rows: in flight together with W's
        // columns (clamped addresses, then a select); storing dY to LDS
        // waits only for the loads issued before the X rows.
        const int nfl = min(kLnbBatch, M - rb0) * N;     // the batch's dY floats
        const float* dyb = dy + (int64_t)rb0 * N;
        float4 dq[kLnbBatch * kLnbMaxN / 4 / 256];
#pragma unroll
        for (int i = 0; i < kLnbBatch * kLnbMaxN / 4 / 256; ++i) {
            const int j = t + 256 * i;
            if (DVEC) {
                const float4 v = *reinterpret_cast<const float4*>(dyb + 4 * min(j, nfl / 4 - 1));
                dq[i] = 4 * j < nfl ? v : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float e4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = dyb[min(4 * j + e, nfl - 1)];
                    e4[e] = 4 * j + e < nfl ? v : 0.0f;
                }
                dq[i] = make_float4(e4[0], e4[1], e4[2], e4[3]);
            }
        }
        float4 xv[kLnbRows];
#pragma unroll
        for (int u = 0; u < kLnbRows; ++u) {
            const int r = rb0 + rg + 16 * u;
            const float4 v = *reinterpret_cast<const float4*>(xb + (int64_t)min(r, M - 1) * xld + kc);
            xv[u] = r < M && colok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (rb0 > 0) __syncthreads();                    // the previous batch's reads are done
#pragma unroll
        for (int i = 0; i < kLnbBatch * kLnbMaxN / 4 / 256; ++i) dys[t + 256 * i] = dq[i];
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kLnbRows; ++u) {
            const int rl = rg + 16 * u, r = rb0 + rl;
            float d[NP];
#pragma unroll
            for (int n = 0; n < NP; ++n) {
                const float v = dyf[rl * N + min(n, N - 1)];
                d[n] = n < N ? v : 0.0f;
            }
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int n = 0; n < NP; ++n) {
                acc[n].x += d[n] * xv[u].x; acc[n].y += d[n] * xv[u].y;
                acc[n].z += d[n] * xv[u].z; acc[n].w += d[n] * xv[u].w;
                o.x += d[n] * wv[n].x; o.y += d[n] * wv[n].y; o.z += d[n] * wv[n].z; o.w += d[n] * wv[n].w;
            }
            if (dx && colok && r < M) *reinterpret_cast<float4*>(dx + (int64_t)r * K + kq) = o;
        }
        if (db && blockIdx.x == 0 && cq < N) {
            // db: thread (column cq, row group rg) adds its rows of the batch.
            // Every row's read is issued and rows past M add +0.0 (no change
            // to a sum that starts at +0.0), so the reads are in flight
            // together instead of one branch and one wait per row.
            float dr[kLnbRows];
#pragma unroll
            for (int u = 0; u < kLnbRows; ++u) dr[u] = dyf[(rg + 16 * u) * N + cq];
#pragma unroll
            for (int u = 0; u < kLnbRows; ++u) dbv += rb0 + rg + 16 * u < M ? dr[u] : 0.0f;
        }
    }
    if (dw) {
#pragma unroll
        for (int n = 0; n < NP; ++n)
            if (n < N) *reinterpret_cast<float4*>(red + (rg * N + n) * kLnbCols + 4 * cq) = acc[n];
        __syncthreads();
        if (t < N * 16) {
            const int n = t >> 4, q = t & 15, k = k0 + 4 * q;
            float4 v = *reinterpret_cast<const float4*>(red + n * kLnbCols + 4 * q);
            for (int g = 1; g < 16; ++g) {
                const float4 a = *reinterpret_cast<const float4*>(red + (g * N + n) * kLnbCols + 4 * q);
                v.x += a.x; v.y += a.y; v.z += a.z; v.w += a.w;
            }
            if (k < K) *reinterpret_cast<float4*>(dw + (int64_t)n * K + k) = v;
        }
    }
    if (db && blockIdx.x == 0) {
        // The 16 row groups' db sums, added in group order.
        __shared__ float dbs[16][kLnbMaxN];
        if (cq < N) dbs[rg][cq] = dbv;
        __syncthreads();
        if (t < N) {
            float v = dbs[0][t];
            for (int g = 1; g < 16; ++g) v += dbs[g][t];
            db[t] = v;
        }
    }
}

size_t linear_bwd_narrow_lds(int64_t N) { return (size_t)(16 * N * kLnbCols) * sizeof(float); }

}  // namespace

namespace tfh {

tf_status sum_partials(tf_ctx* ctx, const float* part, int64_t splits, int64_t M, int64_t N, float* out, int64_t ldc) {
    if (M == 0 || N == 0) return TF_OK;
    GemmParams p{};
    p.partial = const_cast<float*>(part);
    p.C = out;
    p.M = (int)M;
    p.N = (int)N;
    p.ldc = ldc;
    p.alpha = 1.0f;
    p.epi = TF_EPI_NONE;
    splitk_reduce_wide_kernel<<<(unsigned)((M * N + 15) / 16), 256, 0, ctx->stream>>>(p, (int)splits);
    return check_launch("splitk_reduce_wide_kernel");
}

}  // namespace tfh

extern "C" {

tf_status tf_gemm(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                  const void* A, int64_t lda, const void* B, int64_t ldb, float beta, void* C, int64_t ldc,
                  int in_dtype, int out_dtype, int epilogue, const float* bias) {
    tfh::TimedLaunch timed(ctx, M, N, K, 1, trans_a, trans_b, in_dtype, out_dtype);
    return gemm_impl(ctx, trans_a, trans_b, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1, 0,
                     in_dtype, out_dtype, epilogue, bias);
}

tf_status tf_gemm_noalloc(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                          const void* A, int64_t lda, const void* B, int64_t ldb, float beta, void* C, int64_t ldc,
                          int in_dtype, int out_dtype, int epilogue, const float* bias) {
    tfh::TimedLaunch timed(ctx, M, N, K, 1, trans_a, trans_b, in_dtype, out_dtype);
    return gemm_impl(ctx, trans_a, trans_b, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1, 0,
                     in_dtype, out_dtype, epilogue, bias, /*noalloc=*/true);
}

tf_status tf_gemm_strided_batched(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                                  float alpha, const void* A, int64_t lda, int64_t stride_a, const void* B,
                                  int64_t ldb, int64_t stride_b, float beta, void* C, int64_t ldc,
                                  int64_t stride_c, int64_t batch, int in_dtype, int out_dtype) {
    tfh::TimedLaunch timed(ctx, M, N, K, batch, trans_a, trans_b, in_dtype, out_dtype);
    return gemm_impl(ctx, trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                     stride_c, batch, 0, in_dtype, out_dtype, TF_EPI_NONE, nullptr);
}

tf_status tf_gemm_ex(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                     const void* A, int64_t lda, int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b,
                     float beta, void* C, int64_t ldc, int64_t stride_c, int64_t batch, int reduce_batch,
                     int in_dtype, int out_dtype, int epilogue, const float* bias) {
    tfh::TimedLaunch timed(ctx, M, N, K, reduce_batch ? -batch : batch, trans_a, trans_b, in_dtype, out_dtype);
    return gemm_impl(ctx, trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                     stride_c, batch, reduce_batch, in_dtype, out_dtype, epilogue, bias);
}

tf_status tf_gemm_relu_masked(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                              const float* A, int64_t lda, const float* mask, const float* B, int64_t ldb, float* C,
                              int64_t ldc) {
    TF_REQUIRE(mask != nullptr || M == 0 || N == 0, "tf_gemm_relu_masked: null mask");
    tfh::TimedLaunch timed(ctx, M, N, K, 1, trans_a, trans_b, TF_F32, TF_F32);
    return gemm_impl(ctx, trans_a, trans_b, M, N, K, 1.0f, A, lda, 0, B, ldb, 0, 0.0f, C, ldc, 0, 1, 0, TF_F32,
                     TF_F32, TF_EPI_NONE, nullptr, false, mask);
}

tf_status tf_linear_bwd_small(tf_ctx* ctx, const float* dy, const float* mask, const float* x, const float* w,
                              float* dx, float* dw, int64_t M, int64_t N, int64_t K) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31),
               "tf_linear_bwd_small: extents must be positive");
    TF_REQUIRE(dy && x && w && dx && dw, "tf_linear_bwd_small: null pointer");
    // dX = dZ W: M x K over N (A = dZ K-major, B = W rows); dW = dZ^T X:
    // N x K over M (A = dZ read transposed, B = X rows).
    int64_t t1, g1, t2, g2;
    int c1, c2;
    if (!small_grid(ctx->num_cus, M, K, N, t1, g1, c1) || !small_grid(ctx->num_cus, N, K, M, t2, g2, c2) ||
        t1 + t2 > tfh::kTicketGemmTiles)
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_linear_bwd_small: a product does not fit the small-product kernel "
                                                  "(K <= 2048 and M*N*K <= 2^27 for each)");
    auto params = [&](const float* B, float* C, int64_t Mi, int64_t Ni, int64_t Ki) {
        GemmParams q{};
        q.A = dy; q.B = B; q.C = C;
        q.lda = N; q.ldb = K; q.ldc = K;
        q.M = (int)Mi; q.N = (int)Ni; q.K = (int)Ki;
        q.tiles_m = (int)((Mi + kSmT - 1) / kSmT);
        q.tiles_n = (int)((Ni + kSmT - 1) / kSmT);
        q.reduce_batch = 1;
        q.alpha = 1.0f; q.beta = 0.0f; q.epi = TF_EPI_NONE;
        q.vec_a = aligned16(dy) && N % 4 == 0 && (!mask || aligned16(mask));
        q.vec_b = aligned16(B) && K % 4 == 0;
        q.mask_a = mask;
        return q;
    };
    GemmParams p1 = params(w, dx, M, K, N), p2 = params(x, dw, N, K, M);
    const size_t part1 = g1 > 1 ? (size_t)t1 * g1 * kSmT * kSmT * sizeof(float) : 0;
    const size_t part2 = g2 > 1 ? (size_t)t2 * g2 * kSmT * kSmT * sizeof(float) : 0;
    if (part1 + part2 > 0) {
        tf_status st = tfh::ensure_workspace(ctx, part1 + part2);
        if (st != TF_OK) return st;
        p1.partial = reinterpret_cast<float*>(ctx->ws);
        p2.partial = reinterpret_cast<float*>(reinterpret_cast<char*>(ctx->ws) + part1);
    }
    const int blocks1 = (int)(t1 * g1), blocks2 = (int)(t2 * g2);
    unsigned* tickets = ctx->tickets + tfh::kTicketGemm;
    gemm_f32_small_pair_kernel<<<(unsigned)(blocks1 + blocks2), 256, 0, ctx->stream>>>(
        p1, (int)g1, c1, tickets, blocks1, p2, (int)g2, c2, tickets + t1);
    return tfh::check_launch("gemm_f32_small_pair_kernel");
}

tf_status tf_linear_bwd_narrow(tf_ctx* ctx, const float* dy, const float* x, const float* w, float* dx, float* dw,
                               float* db, int64_t M, int64_t N, int64_t K) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(M >= 0 && N >= 1 && N <= kLnbMaxN && K >= 0 && K % 4 == 0 && K < (1LL << 31) && M * K < (1LL << 40),
               "tf_linear_bwd_narrow: needs 1 <= N <= 16 outputs and K % 4 == 0");
    if (M == 0 || K == 0) {
        if (dw) { tf_status st = tf_hip_fill_f32(ctx, dw, 0.0f, N * K); if (st != TF_OK) return st; }
        if (db) return tf_hip_fill_f32(ctx, db, 0.0f, N);
        return TF_OK;
    }
    TF_REQUIRE(dy && w && (x || !dw), "tf_linear_bwd_narrow: null pointer");
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    TF_REQUIRE(a16(w) && (!x || a16(x)) && (!dx || a16(dx)) && (!dw || a16(dw)),
               "tf_linear_bwd_narrow: x, w, dx and dw must be 16-byte aligned");
    static const bool lds_ok = [] {
        const void* fns[] = {
            reinterpret_cast<const void*>(linear_bwd_narrow_kernel<4, true>),
            reinterpret_cast<const void*>(linear_bwd_narrow_kernel<8, true>),
            reinterpret_cast<const void*>(linear_bwd_narrow_kernel<12, true>),
            reinterpret_cast<const void*>(linear_bwd_narrow_kernel<16, true>),
            reinterpret_cast<const void*>(linear_bwd_narrow_kernel<4, false>),
            reinterpret_cast<const void*>(linear_bwd_narrow_kernel<8, false>),
            reinterpret_cast<const void*>(linear_bwd_narrow_kernel<12, false>),
            reinterpret_cast<const void*>(linear_bwd_narrow_kernel<16, false>)};
        for (const void* f : fns)
            if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)linear_bwd_narrow_lds(kLnbMaxN)) != hipSuccess)
                return false;
        return true;
    }();
    if (!lds_ok) {
        (void)hipGetLastError();
        return tfh::set_error(TF_ERR_HIP, "tf_linear_bwd_narrow: hipFuncSetAttribute (dynamic LDS) failed");
    }
    const unsigned blocks = (unsigned)((K + kLnbCols - 1) / kLnbCols);
    const size_t lds = dw ? linear_bwd_narrow_lds(N) : 0;
    const int np = (int)((N + 3) / 4 * 4);
    const bool dvec = (M * N) % 4 == 0 && (reinterpret_cast<uintptr_t>(dy) & 15) == 0;
#define TF_LNB_LAUNCH(NPV)                                                                                       \
    do {                                                                                                         \
        if (dvec)                                                                                                \
            linear_bwd_narrow_kernel<NPV, true><<<blocks, 256, lds, ctx->stream>>>(dy, x, w, dx, dw, db, (int)M, \
                                                                                   (int)N, (int)K);              \
        else                                                                                                     \
            linear_bwd_narrow_kernel<NPV, false><<<blocks, 256, lds, ctx->stream>>>(dy, x, w, dx, dw, db,        \
                                                                                    (int)M, (int)N, (int)K);     \
    } while (0)
    if (np == 4) TF_LNB_LAUNCH(4);
    else if (np == 8) TF_LNB_LAUNCH(8);
    else if (np == 12) TF_LNB_LAUNCH(12);
    else TF_LNB_LAUNCH(16);
#undef TF_LNB_LAUNCH
    return tfh::check_launch("linear_bwd_narrow_kernel");
}

}  // extern "C"
