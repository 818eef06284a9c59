// Fused NF4 dequant-GEMMs for gfx950 (bf16 / fp16 MFMA, fp32 accumulate).
//
// forward  Y[M, N]  = X[M, K] . W[N, K]^T  (+ bias) (+ T . L^T)
// backward dX[M, K] = dY[M, N] . W[N, K]            (+ U . At^T)
//
// Work-group tile 128 x 128, 4 waves in a 2 x 2 grid, each wave 64 x 64 as
// 2 x 2 v_mfma_f32_32x32x16 tiles; the reduction advances 64 at a time (one
// NF4 block of 64 when blocksize = 64). Per step the activation tile is copied
// to LDS and the packed W tile is dequantized (level table in LDS, fp32
// product with the block absmax, one round-to-nearest-even conversion: the
// same values the dequantize kernel writes) straight into LDS, so every
// dequantized element is reused by 128 rows of activations. LDS rows are
// 64 halfs (128 B = eight 16-byte chunks); chunk c of row r lives at
// c ^ (r & 7), which makes both the 16-byte fragment reads of the MFMA loop
// and the 16-byte tile writes bank-conflict free. Two LDS buffers: the global
// loads of step k+1 are in flight while the MFMAs of step k run.
//
// MFMA operand layout (v_mfma_f32_32x32x16_{bf16,f16}): lane l supplies
// A[l % 32][8 (l / 32) .. +8] and B[8 (l / 32) .. +8][l % 32]; the 16 results of
// lane l are C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32], v = 0..15.
#include <type_traits>

#include "nf4_kernels.h"

namespace stm {

namespace {

constexpr int BM = 128;   // rows of the activation / output tile
constexpr int BN = 128;   // output columns per tile
constexpr int BK = 64;    // reduction step
constexpr int NT = 256;   // threads

template <typename Tr>
__device__ __forceinline__ f32x16_t mfma(const uint4& a, const uint4& b, const f32x16_t& c) {
    if constexpr (Tr::tag == STM_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                      0, 0, 0);
}

__device__ __forceinline__ int swz(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

// Group bookkeeping: expert e owns rows [row0, row0 + rows) of a/out and the
// e-th [N, K] slice of the packed weight.
struct Group {
    int64_t row0, rows;
    const uint8_t* packed;
    const float* absmax;
};

__device__ __forceinline__ Group group_of(const GemmArgs& g, int e) {
    Group r;
    if (g.offsets) {
        r.row0 = g.offsets[e];
        r.rows = (int64_t)g.offsets[e + 1] - r.row0;
    } else {
        r.row0 = 0;
        r.rows = g.M;
    }
    const int64_t wnum = g.N * g.K;
    r.packed = g.packed + (int64_t)e * (wnum / 2);
    r.absmax = g.absmax + (int64_t)e * (wnum / g.blocksize);
    return r;
}

// One packed byte -> two dequantized 16-bit values (even element in the low half).
template <typename Tr>
__device__ __forceinline__ uint32_t deq2(const float2* __restrict__ lut, uint32_t byte, float a) {
    const float2 c = lut[byte];
    return Tr::pack2(opaque(c.x * a), opaque(c.y * a));
}

// Rank-R epilogue term: acc[i][j] += A_r[rows] . B_r[cols]^T, both operands
// row-major with R contiguous (rows of the lora_x / lora_w matrices).
template <typename Tr>
__device__ __forceinline__ void lora_term(f32x16_t (&acc)[2][2], const uint16_t* __restrict__ ax, int64_t row_base,
                                          int64_t rows_valid, const uint16_t* __restrict__ bw, int64_t col_base,
                                          int64_t cols_valid, int R, int lane) {
    for (int r0 = 0; r0 < R; r0 += 16) {
        uint4 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t row = row_base + i * 32 + (lane & 31);
            a[i] = make_uint4(0, 0, 0, 0);
            if (row < rows_valid) a[i] = *reinterpret_cast<const uint4*>(ax + row * R + r0 + 8 * (lane >> 5));
            const int64_t col = col_base + i * 32 + (lane & 31);
            b[i] = make_uint4(0, 0, 0, 0);
            if (col < cols_valid) b[i] = *reinterpret_cast<const uint4*>(bw + col * R + r0 + 8 * (lane >> 5));
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = mfma<Tr>(a[i], b[j], acc[i][j]);
    }
}

template <typename Tr>
__device__ __forceinline__ void store_tile(const f32x16_t (&acc)[2][2], uint16_t* __restrict__ out, int64_t ld,
                                           int64_t row_base, int64_t rows_valid, int64_t col_base, int64_t cols_valid,
                                           const uint16_t* __restrict__ bias, int lane) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int64_t col = col_base + j * 32 + (lane & 31);
        if (col >= cols_valid) continue;
        const float bv = bias ? Tr::to_f32(bias[col]) : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t row = row_base + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (row < rows_valid) out[row * ld + col] = Tr::from_f32(acc[i][j][v] + bv);
            }
        }
    }
}

// ------------------------------------------------------------------ forward
template <typename Tr>
__global__ __launch_bounds__(NT) void k_gemm_fwd(GemmArgs g) {
    __shared__ uint4 sA[2][BM * 8];
    __shared__ uint4 sB[2][BN * 8];
    __shared__ float2 lut[256];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    lut[tid] = make_float2(kLevelsDev[tid >> 4], kLevelsDev[tid & 15]);

    const Group grp = group_of(g, blockIdx.y);
    const int64_t ntn = (g.N + BN - 1) / BN;
    const int64_t m0 = (int64_t)(blockIdx.x / ntn) * BM;
    const int64_t n0 = (int64_t)(blockIdx.x % ntn) * BN;
    if (m0 >= grp.rows) return;

    const uint16_t* __restrict__ X = reinterpret_cast<const uint16_t*>(g.a) + grp.row0 * g.K;
    const int64_t K = g.K, N = g.N;
    const int64_t kblocks = K / g.blocksize;
    const int bshift = ilog2(g.blocksize);

    // this thread's slice of the tiles
    const int xa_row = tid >> 3, xa_chunk = tid & 7;     // + 32 * i, i = 0..3
    const int wb_row = tid >> 1, wb_half = tid & 1;      // 16 packed bytes = 32 elements
    const int64_t w_row = n0 + wb_row;
    const bool w_ok = w_row < N;
    const uint8_t* __restrict__ wp = grp.packed + w_row * (K / 2) + wb_half * 16;
    const float* __restrict__ wa = grp.absmax + w_row * kblocks;

    uint4 xr[4], wr;
    float ar;
    auto gload = [&](int kt) {
        const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t row = m0 + xa_row + 32 * i;
            xr[i] = make_uint4(0, 0, 0, 0);
            if (row < grp.rows) xr[i] = *reinterpret_cast<const uint4*>(X + row * K + k0 + xa_chunk * 8);
        }
        wr = make_uint4(0, 0, 0, 0);
        ar = 0.0f;
        if (w_ok) {
            wr = *reinterpret_cast<const uint4*>(wp + k0 / 2);
            ar = wa[k0 >> bshift];
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sA[buf][swz(xa_row + 32 * i, xa_chunk)] = xr[i];
        const uint32_t w4[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // packed word c -> 8 elements -> one 16-byte chunk
            uint4 o;
            o.x = deq2<Tr>(lut, w4[c] & 0xFFu, ar);
            o.y = deq2<Tr>(lut, (w4[c] >> 8) & 0xFFu, ar);
            o.z = deq2<Tr>(lut, (w4[c] >> 16) & 0xFFu, ar);
            o.w = deq2<Tr>(lut, w4[c] >> 24, ar);
            sB[buf][swz(wb_row, wb_half * 4 + c)] = o;
        }
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int KT = (int)(K / BK);
    gload(0);
    __syncthreads();  // lut ready
    lstore(0);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            uint4 a[2], b[2];
            const int ch = kk * 2 + (lane >> 5);
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = sA[cur][swz(wm * 64 + i * 32 + (lane & 31), ch)];
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = sB[cur][swz(wn * 64 + j * 32 + (lane & 31), ch)];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma<Tr>(a[i], b[j], acc[i][j]);
        }
        if (kt + 1 < KT) lstore(cur ^ 1);
        __syncthreads();
    }

    const int64_t row_base = m0 + wm * 64, col_base = n0 + wn * 64;
    if (g.lora_rank > 0)
        lora_term<Tr>(acc, reinterpret_cast<const uint16_t*>(g.lora_x) + grp.row0 * g.lora_rank, row_base, grp.rows,
                      reinterpret_cast<const uint16_t*>(g.lora_w), col_base, N, g.lora_rank, lane);
    store_tile<Tr>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * N, N, row_base, grp.rows, col_base, N,
                   reinterpret_cast<const uint16_t*>(g.bias), lane);
}

// ----------------------------------------------------------------- backward
// dX[m, k] = sum_n dY[m, n] W[n, k]: the W tile (64 rows n x 128 columns k) is
// dequantized transposed into LDS as [k][n] so the MFMA B operand (8
// consecutive n per lane) is one 16-byte read.
template <typename Tr>
__global__ __launch_bounds__(NT) void k_gemm_bwd(GemmArgs g) {
    constexpr int BKO = 128;  // output columns (k) per tile
    constexpr int BR = 64;    // reduction step over n
    __shared__ uint4 sA[2][BM * 8];
    __shared__ uint4 sB[2][BKO * 8];
    __shared__ float2 lut[256];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wk = wave & 1;
    lut[tid] = make_float2(kLevelsDev[tid >> 4], kLevelsDev[tid & 15]);

    const Group grp = group_of(g, blockIdx.y);
    const int64_t K = g.K, N = g.N;
    const int64_t ntk = (K + BKO - 1) / BKO;
    const int64_t m0 = (int64_t)(blockIdx.x / ntk) * BM;
    const int64_t k0 = (int64_t)(blockIdx.x % ntk) * BKO;
    if (m0 >= grp.rows) return;

    const uint16_t* __restrict__ DY = reinterpret_cast<const uint16_t*>(g.a) + grp.row0 * N;
    const int64_t kblocks = K / g.blocksize;
    const int bshift = ilog2(g.blocksize);

    const int xa_row = tid >> 3, xa_chunk = tid & 7;
    // W slice: 8 rows (n-group ng) x 4 columns (k-group kg)
    const int ng = tid & 7, kg = tid >> 3;
    const int64_t wk_col = k0 + kg * 4;
    const bool wk_ok = wk_col < K;
    const int64_t wk_blk = wk_col >> bshift;

    uint4 xr[4];
    uint32_t wr[8];
    float ar[8];
    auto gload = [&](int nt) {
        const int64_t n0 = (int64_t)nt * BR;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t row = m0 + xa_row + 32 * i;
            xr[i] = make_uint4(0, 0, 0, 0);
            if (row < grp.rows) xr[i] = *reinterpret_cast<const uint4*>(DY + row * N + n0 + xa_chunk * 8);
        }
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int64_t n = n0 + ng * 8 + r;  // N % 64 == 0: always < N
            wr[r] = 0u;
            ar[r] = 0.0f;
            if (wk_ok) {
                wr[r] = *reinterpret_cast<const uint16_t*>(grp.packed + n * (K / 2) + wk_col / 2);
                ar[r] = grp.absmax[n * kblocks + wk_blk];
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sA[buf][swz(xa_row + 32 * i, xa_chunk)] = xr[i];
        // element (row r, column c) of the 8x4 slice: byte c/2 of wr[r], high nibble for even c
        float v[4][8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const float2 lo = lut[wr[r] & 0xFFu], hi = lut[(wr[r] >> 8) & 0xFFu];
            v[0][r] = opaque(lo.x * ar[r]);
            v[1][r] = opaque(lo.y * ar[r]);
            v[2][r] = opaque(hi.x * ar[r]);
            v[3][r] = opaque(hi.y * ar[r]);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint4 o;
            o.x = Tr::pack2(v[c][0], v[c][1]);
            o.y = Tr::pack2(v[c][2], v[c][3]);
            o.z = Tr::pack2(v[c][4], v[c][5]);
            o.w = Tr::pack2(v[c][6], v[c][7]);
            sB[buf][swz(kg * 4 + c, ng)] = o;
        }
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int NTILES = (int)(N / BR);
    gload(0);
    __syncthreads();
    lstore(0);
    __syncthreads();

    for (int nt = 0; nt < NTILES; ++nt) {
        const int cur = nt & 1;
        if (nt + 1 < NTILES) gload(nt + 1);
#pragma unroll
        for (int kk = 0; kk < BR / 16; ++kk) {
            uint4 a[2], b[2];
            const int ch = kk * 2 + (lane >> 5);
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = sA[cur][swz(wm * 64 + i * 32 + (lane & 31), ch)];
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = sB[cur][swz(wk * 64 + j * 32 + (lane & 31), ch)];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma<Tr>(a[i], b[j], acc[i][j]);
        }
        if (nt + 1 < NTILES) lstore(cur ^ 1);
        __syncthreads();
    }

    const int64_t row_base = m0 + wm * 64, col_base = k0 + wk * 64;
    if (g.lora_rank > 0)
        lora_term<Tr>(acc, reinterpret_cast<const uint16_t*>(g.lora_x) + grp.row0 * g.lora_rank, row_base, grp.rows,
                      reinterpret_cast<const uint16_t*>(g.lora_w), col_base, K, g.lora_rank, lane);
    store_tile<Tr>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * K, K, row_base, grp.rows, col_base, K,
                   nullptr, lane);
}

}  // namespace

int launch_gemm_fwd(const GemmArgs& g, int dtype, hipStream_t stream) {
    const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    if (tiles == 0) return STM_OK;
    if (tiles > 0x7FFFFFFFLL || g.num_groups > 65535) return set_error(STM_ERR_UNSUPPORTED, "gemm_fwd: grid too large");
    dim3 grid((unsigned)tiles, (unsigned)g.num_groups), block(NT);
    if (dtype == STM_BF16)
        hipLaunchKernelGGL(k_gemm_fwd<BF16>, grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL(k_gemm_fwd<F16>, grid, block, 0, stream, g);
    return check_launch("gemm_fwd");
}

int launch_gemm_bwd(const GemmArgs& g, int dtype, hipStream_t stream) {
    const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.K + 127) / 128);
    if (tiles == 0) return STM_OK;
    if (tiles > 0x7FFFFFFFLL || g.num_groups > 65535)
        return set_error(STM_ERR_UNSUPPORTED, "gemm_bwd_dx: grid too large");
    dim3 grid((unsigned)tiles, (unsigned)g.num_groups), block(NT);
    if (dtype == STM_BF16)
        hipLaunchKernelGGL(k_gemm_bwd<BF16>, grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL(k_gemm_bwd<F16>, grid, block, 0, stream, g);
    return check_launch("gemm_bwd_dx");
}

}  // namespace stm
