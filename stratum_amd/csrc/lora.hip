// Rank-R side products of a LoRA adapter on a frozen base (gfx950).
//
// PEFT's lora.Linear adds s * (X A^T) B^T to the frozen projection; its autograd
// then needs, besides the base input gradient:
//
//   forward   T  = s * X  A^T    [M, R]   (X [M, K], A [R, K])
//   backward  U  = s * dY B      [M, R]   (dY [M, N], B [N, R])
//             dB = dY^T T        [N, R]
//             dA = U^T X         [R, K]
//
// Each reads one large operand (X or dY) and is bound by HBM bandwidth: 2 bytes
// per element of X or dY, R * 2 flops per element and product. One kernel
// covers all four. It streams Z (X or dY, row-major [rows, cols]) through LDS,
// 64 rows x 256 columns per step, and contracts each tile two ways with
// v_mfma_f32_16x16x32:
//
//   ROW  out_row[m, r] = sum_c Z[m, c] P[c, r]   (T: P = A^T;  U: P = B)
//   COL  out_col[c, r] = sum_m Z[m, c] Q[m, r]   (dB: Q = T;   dA^T: Q = U)
//
// so the backward reads dY once for U and dB. A work-group owns 256 columns and
// a range of rows. Its ROW sums cover only its own columns, and its COL sums only
// its own rows. Both go to fp32 partial buffers ([column block][m][r] and
// [row block][c][r]). A second kernel adds the partials in a fixed order, scales
// and rounds once to bf16/fp16, so results do not depend on scheduling.
//
// MFMA operand layout (16x16x32): lane l holds 8 consecutive reduction indices
// 8 (l / 16) + (0..7) of row (A) or column (B) l % 16, and the result D[i][j]
// sits in lane j + 16 (i / 4), element i % 4. The reduction index of ROW is the
// column of Z (contiguous: one 16-byte LDS read per operand); that of COL is the
// row of Z, so its Z operand is gathered from LDS as 8 16-bit values. The small
// operands P (per work-group) and Q (per step) are staged in LDS transposed,
// [rank][index] with 16 bytes of padding per rank row, so both MFMA sides read
// 16-byte runs.
#include <initializer_list>

#include "nf4_common.h"

namespace stm {
namespace {

constexpr int LR_TN = 256;  // columns of Z per work-group
constexpr int LR_SM = 64;   // rows of Z per step
constexpr int LR_CH = LR_TN / 8;   // 16-byte chunks per tile row
constexpr int LR_PS = LR_TN + 8;   // bf16 stride of a staged P rank row (528 bytes)
constexpr int LR_QS = LR_SM + 8;   // bf16 stride of a staged Q rank row (144 bytes)

// Chunk swizzle of the Z tile (tile row m, 16-byte chunk q at q ^ zswz(m)). The
// ROW reads take one chunk of 16 consecutive rows; the COL gathers take two
// adjacent chunks of the rows 8 apart. Both then hit distinct bank groups.
__device__ __forceinline__ int zswz(int m) { return (m & 15) ^ (((m >> 3) & 3) << 1); }

typedef short s16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

template <typename Tr>
__device__ __forceinline__ f32x4_t mfma16x32(const uint4& a, const uint4& b, const f32x4_t& c) {
    if constexpr (Tr::tag == STM_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

struct LoraArgs {
    const uint16_t* z;  // [rows, cols]
    const uint16_t* p;  // ROW operand: [cols, R] (p_t = 0) or [R, cols] (p_t = 1)
    const uint16_t* q;  // COL operand: [rows, R]
    float* part_row;    // [column blocks][rows][RP]
    float* part_col;    // [row blocks][cols][RP]
    int64_t rows, cols;
    int rank;           // R (a multiple of 8)
    int p_t;
    int rows_per_block; // a multiple of LR_SM
};

// RP = R rounded up to 16 (zero ranks padded). ROW / COL select the products.
template <typename Tr, int RP, bool ROW, bool COL>
__global__ __launch_bounds__(256, 2) void k_lora_pass(LoraArgs g) {
    constexpr int G = RP / 16;  // rank groups of 16
    __shared__ uint4 zt[LR_SM * LR_CH];                   // 32 KB
    __shared__ __attribute__((aligned(16))) uint16_t ps[ROW ? RP * LR_PS : 8];  // P^T block [RP][256 (+8)]
    __shared__ __attribute__((aligned(16))) uint16_t qs[COL ? RP * LR_QS : 8];  // Q^T of the step [RP][64 (+8)]

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lh = lane >> 4;
    const int64_t cb = blockIdx.x, rb = blockIdx.y;
    const int64_t c0 = cb * LR_TN;
    const int64_t m_begin = rb * g.rows_per_block;
    const int64_t m_end = m_begin + g.rows_per_block < g.rows ? m_begin + g.rows_per_block : g.rows;
    const int R = g.rank;

    if constexpr (ROW) {
        // P^T [RP][256]: zero outside the matrix and for ranks >= R
        if (g.p_t) {
            for (int i = tid; i < RP * LR_CH; i += 256) {
                const int r = i / LR_CH, q = i % LR_CH;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (r < R && c0 + 8 * q < g.cols) v = *reinterpret_cast<const uint4*>(g.p + r * g.cols + c0 + 8 * q);
                *reinterpret_cast<uint4*>(ps + r * LR_PS + 8 * q) = v;
            }
        } else {
            for (int i = tid; i < LR_TN * (RP / 8); i += 256) {
                const int c = i / (RP / 8), r8 = i % (RP / 8);
                uint4 v = make_uint4(0, 0, 0, 0);
                if (8 * r8 < R && c0 + c < g.cols) v = *reinterpret_cast<const uint4*>(g.p + (c0 + c) * R + 8 * r8);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    ps[(8 * r8 + 2 * j) * LR_PS + c] = (uint16_t)(w[j] & 0xFFFFu);
                    ps[(8 * r8 + 2 * j + 1) * LR_PS + c] = (uint16_t)(w[j] >> 16);
                }
            }
        }
    }

    // Z tile of one step: thread t takes chunks t + 256 i (row 8 i + t / 32, chunk
    // t % 32); Q rows of the step, 8 ranks per thread. Rows past the work-group's
    // range and columns past the matrix load as zeros, so the loads of a step
    // beyond the range are harmless (and keep the wait counts uniform).
    struct Regs {
        uint4 z[8];
        uint4 q;
    };
    // Buffer loads: the resource spans the work-group's rows, so a row past its
    // range reads as zero by the hardware range check, and a column past the
    // matrix gets an offset beyond the range. No branch around a load, so the
    // compiler's wait counts stay exact. (Offsets stay below 2^32: the host
    // keeps rows_per_block * cols * 2 below 2^31 and cols below 2^22.)
    constexpr uint32_t kOut = 0x80000000u;
    const uint32_t zrow = (uint32_t)g.cols * 2u;
    const __amdgpu_buffer_rsrc_t zres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(g.z + m_begin * g.cols), (short)0, (int)((m_end - m_begin) * (int64_t)zrow), 0x00020000);
    const int zq = tid & 31;
    const uint32_t zlane = c0 + 8 * zq < g.cols ? (uint32_t)(tid >> 5) * zrow + (uint32_t)(c0 + 8 * zq) * 2u : kOut;
    const uint32_t qrow = (uint32_t)R * 2u;
    const __amdgpu_buffer_rsrc_t qres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(COL ? g.q + m_begin * R : g.z), (short)0, COL ? (int)((m_end - m_begin) * (int64_t)qrow) : 0,
        0x00020000);
    // this column block's ROW partials [rows][RP] (without ROW an empty range:
    // every store through it is dropped)
    const __amdgpu_buffer_rsrc_t pres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(ROW ? g.part_row + cb * g.rows * RP : g.part_col), (short)0, ROW ? (int)(g.rows * RP * 4) : 0,
        0x00020000);
    const int qm = tid / (RP / 8), qr8 = tid % (RP / 8);
    const bool qlane = tid < LR_SM * (RP / 8);
    const uint32_t qlane_off = (qlane && 8 * qr8 < R) ? (uint32_t)qm * qrow + 16u * (uint32_t)qr8 : kOut;
    auto load = [&](int64_t m0, Regs& r) {
        const uint32_t step = (uint32_t)(m0 - m_begin);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t off = zlane == kOut ? kOut : zlane + (step + 8u * i) * zrow;
            r.z[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(zres, (int)off, 0, 0));
        }
        if constexpr (COL) {
            const uint32_t off = qlane_off == kOut ? kOut : qlane_off + step * qrow;
            r.q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qres, (int)off, 0, 0));
        }
    };
    auto stage = [&](const Regs& r) {
        const int q = tid & 31;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int m = 8 * i + (tid >> 5);
            zt[m * LR_CH + (q ^ zswz(m))] = r.z[i];
        }
        if constexpr (COL) {
            if (qlane) {
                const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    qs[(8 * qr8 + 2 * j) * LR_QS + qm] = (uint16_t)(w[j] & 0xFFFFu);
                    qs[(8 * qr8 + 2 * j + 1) * LR_QS + qm] = (uint16_t)(w[j] >> 16);
                }
            }
        }
    };

    const __attribute__((address_space(3))) uint4* lds_zt = (const __attribute__((address_space(3))) uint4*)zt;
    f32x4_t acc_col[4][G];
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int k = 0; k < G; ++k) acc_col[f][k] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // products of the staged step starting at row m0
    auto compute = [&](int64_t m0) {
        if constexpr (ROW) {
            // wave w: tile rows 16 w .. 16 w + 15 against all 256 columns
            f32x4_t acc[G];
#pragma unroll
            for (int k = 0; k < G; ++k) acc[k] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            const int m = 16 * wave + lr;
#pragma unroll
            for (int kc = 0; kc < LR_CH / 4; ++kc) {
                const uint4 b = zt[m * LR_CH + ((4 * kc + lh) ^ zswz(m))];
#pragma unroll
                for (int k = 0; k < G; ++k) {
                    const uint4 a = *reinterpret_cast<const uint4*>(ps + (16 * k + lr) * LR_PS + 32 * kc + 8 * lh);
                    acc[k] = mfma16x32<Tr>(a, b, acc[k]);
                }
            }
            // buffer stores: a row past the range gets an offset the range check drops
            const int64_t om = m0 + m;
            const uint32_t off = om < m_end ? (uint32_t)(om * RP * 4) + 16u * lh : kOut;
#pragma unroll
            for (int k = 0; k < G; ++k)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, acc[k]), pres,
                                                       (int)(off == kOut ? kOut : off + 64u * k), 0, 0);
        }
        if constexpr (COL) {
            // wave w: tile columns 64 w .. 64 w + 63 (four groups of 16) against
            // the step's 64 rows (two reduction chunks of 32)
#pragma unroll
            for (int mc = 0; mc < 2; ++mc) {
                uint4 a[G];
#pragma unroll
                for (int k = 0; k < G; ++k)
                    a[k] = *reinterpret_cast<const uint4*>(qs + (16 * k + lr) * LR_QS + 32 * mc + 8 * lh);
#pragma unroll
                for (int f = 0; f < 4; ++f) {
                    // lane lr needs rows 32 mc + 8 lh + 0..7 of column 64 w + 16 f + lr:
                    // two transposed reads of 4 rows x 16 columns, in which lane s of
                    // the 16-lane group points at 4 columns 4 (s % 4) .. of row s / 4
                    // and receives column s of the 4 rows (gfx950 lane layout)
                    const int tc = 64 * wave + 16 * f + 4 * (lr & 3);
                    uint2 half[2];
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int m = 32 * mc + 8 * lh + 4 * hh + (lr >> 2);
                        const uint32_t byte = (uint32_t)((m * LR_CH + ((tc >> 3) ^ zswz(m))) * 16 + (tc & 7) * 2);
                        const s16x4_t t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (__attribute__((address_space(3))) s16x4_t*)((__attribute__((address_space(3))) char*)
                                                                             lds_zt + byte));
                        half[hh] = __builtin_bit_cast(uint2, t);
                    }
                    const uint4 b = make_uint4(half[0].x, half[0].y, half[1].x, half[1].y);
#pragma unroll
                    for (int k = 0; k < G; ++k) acc_col[f][k] = mfma16x32<Tr>(a[k], b, acc_col[f][k]);
                }
            }
        }
    };

    // Two register sets, two steps of loads in flight. Step s: stage its set in
    // LDS, refill the set with step s + 2, compute step s and store its ROW
    // partials (without ROW: stores that the range check drops). The prologue
    // follows each set's loads with as many dropped stores, so the compiler's
    // wait before a stage leaves the other set in flight.
    auto dummy_stores = [&]() {
#pragma unroll
        for (int k = 0; k < G; ++k)
            __builtin_amdgcn_raw_buffer_store_b128(u32x4v{0u, 0u, 0u, 0u}, pres, (int)kOut, 0, 0);
    };
    Regs r0, r1;
    load(m_begin, r0);
    dummy_stores();
    load(m_begin + LR_SM, r1);
    dummy_stores();
    for (int64_t m0 = m_begin; m0 < m_end; m0 += 2 * LR_SM) {
        stage(r0);
        __syncthreads();  // step m0 (and, on the first step, P) published
        load(m0 + 2 * LR_SM, r0);
        compute(m0);
        if constexpr (!ROW) dummy_stores();
        __syncthreads();  // every wave is done with the tile
        stage(r1);
        __syncthreads();
        load(m0 + 3 * LR_SM, r1);
        compute(m0 + LR_SM);
        if constexpr (!ROW) dummy_stores();
        __syncthreads();
    }
    if constexpr (COL) {
        // a work-group with no rows stores zeros, so the reduce can sum every block
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const int64_t c = c0 + 64 * wave + 16 * f + lr;
            if (c < g.cols) {
                float* dst = g.part_col + (rb * g.cols + c) * RP + 4 * lh;
#pragma unroll
                for (int k = 0; k < G; ++k)
                    *reinterpret_cast<float4*>(dst + 16 * k) =
                        make_float4(acc_col[f][k][0], acc_col[f][k][1], acc_col[f][k][2], acc_col[f][k][3]);
            }
        }
    }
}

// One reduction of a launch: out = scale * sum_p part[p][i][r] for i < items,
// r < R, rounded once, over `grid` work-groups.
struct RedJob {
    const float* part;
    int blocks;
    int64_t items;
    float scale;
    uint16_t* out;
    unsigned grid;
};

// out is [items, R] or, with TR, [R, items]. Up to two independent jobs per
// launch (U and dB of one pass): work-groups [0, j0.grid) run j0, the rest j1.
// A work-group takes 64 four-rank vectors; its four waves sum the blocks
// p = w, w + 4, ... (four loads in flight), and wave 0 adds the four sums in
// wave order: a fixed order, so the result does not depend on scheduling.
template <typename Tr, bool TR>
__global__ __launch_bounds__(256) void k_lora_reduce(RedJob j0, RedJob j1, int rank, int rp) {
    const bool second = blockIdx.x >= j0.grid;
    const RedJob& j = second ? j1 : j0;
    const float* __restrict__ part = j.part;
    const int blocks = j.blocks;
    const int64_t items = j.items;
    const float scale = j.scale;
    uint16_t* __restrict__ out = j.out;
    __shared__ float4 sums[4][64];
    const int per = rank / 4;
    const int64_t total = items * per;
    const int il = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t v = (int64_t)(blockIdx.x - (second ? j0.grid : 0u)) * 64 + il;
    const bool live = v < total;
    const int64_t i = live ? v / per : 0;
    const int r = live ? 4 * (int)(v - i * per) : 0;
    const float* src = part + i * rp + r;
    const int64_t bstride = items * rp;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    int p = w;
    for (; p + 12 < blocks; p += 16) {
        float4 t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) t[u] = *reinterpret_cast<const float4*>(src + (int64_t)(p + 4 * u) * bstride);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            s.x += t[u].x;
            s.y += t[u].y;
            s.z += t[u].z;
            s.w += t[u].w;
        }
    }
    for (; p < blocks; p += 4) {
        const float4 t = *reinterpret_cast<const float4*>(src + (int64_t)p * bstride);
        s.x += t.x;
        s.y += t.y;
        s.z += t.z;
        s.w += t.w;
    }
    sums[w][il] = s;
    __syncthreads();
    if (w == 0 && live) {
        float4 a = sums[0][il];
#pragma unroll
        for (int k = 1; k < 4; ++k) {
            const float4 b = sums[k][il];
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        const float o[4] = {a.x * scale, a.y * scale, a.z * scale, a.w * scale};
        if constexpr (TR) {
#pragma unroll
            for (int j = 0; j < 4; ++j) out[(int64_t)(r + j) * items + i] = Tr::from_f32(o[j]);
        } else {
            *reinterpret_cast<uint2*>(out + i * rank + r) = make_uint2(Tr::pack2(o[0], o[1]), Tr::pack2(o[2], o[3]));
        }
    }
}

// T = scaling * X . A^T for at most kDownRowsMax rows (decode sizes): one
// launch, one work-group per row, no workspace (the pass + reduce pair costs
// two launches). Thread j takes the 8-element pieces k = 8 j + 2048 i of the
// row and of every A row (16-byte loads), fp32 products summed per thread in k
// order; the 256 partial vectors meet in LDS in a fixed tree order, and the
// row's R values are scaled and rounded once.
constexpr int64_t kDownRowsMax = 64;
template <typename Tr, int R>
__global__ __launch_bounds__(256) void k_lora_down_rows(const uint16_t* __restrict__ X,
                                                        const uint16_t* __restrict__ A, uint16_t* __restrict__ T,
                                                        int64_t K, float scaling) {
    __shared__ float red[256][R + 1];  // odd row stride: the tree's reads spread over the banks
    const int tid = threadIdx.x;
    const int64_t m = blockIdx.x;
    const uint16_t* x = X + m * K;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    auto unpack = [](const uint4& v, float (&f)[8]) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            f[2 * e] = Tr::to_f32((uint16_t)(w[e] & 0xFFFFu));
            f[2 * e + 1] = Tr::to_f32((uint16_t)(w[e] >> 16));
        }
    };
    for (int64_t k = 8 * (int64_t)tid; k < K; k += 2048) {
        float xf[8];
        unpack(*reinterpret_cast<const uint4*>(x + k), xf);
        uint4 av[R];
#pragma unroll
        for (int r = 0; r < R; ++r) av[r] = *reinterpret_cast<const uint4*>(A + (int64_t)r * K + k);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float af[8];
            unpack(av[r], af);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[r] += xf[e] * af[e];
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) red[tid][r] = acc[r];
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (tid < h) {
#pragma unroll
            for (int r = 0; r < R; ++r) red[tid][r] += red[tid + h][r];
        }
        __syncthreads();
    }
    if (tid < R) T[m * R + tid] = Tr::from_f32(red[0][tid] * scaling);
}

template <typename Tr>
void launch_down_rows(const void* X, const void* A, void* T, int64_t M, int64_t K, int R, float scaling,
                      hipStream_t st) {
    const dim3 grid((unsigned)M), block(256);
    const auto* x = (const uint16_t*)X;
    const auto* a = (const uint16_t*)A;
    auto* t = (uint16_t*)T;
    switch (R) {
        case 8: hipLaunchKernelGGL((k_lora_down_rows<Tr, 8>), grid, block, 0, st, x, a, t, K, scaling); break;
        case 16: hipLaunchKernelGGL((k_lora_down_rows<Tr, 16>), grid, block, 0, st, x, a, t, K, scaling); break;
        case 24: hipLaunchKernelGGL((k_lora_down_rows<Tr, 24>), grid, block, 0, st, x, a, t, K, scaling); break;
        default: hipLaunchKernelGGL((k_lora_down_rows<Tr, 32>), grid, block, 0, st, x, a, t, K, scaling); break;
    }
}

int rank_padded(int R) { return R <= 16 ? 16 : 32; }

// Blocks over the rows: about two work-groups per CU of MI355X's 256 in total,
// three for the row-and-column pass at ranks up to 16 (three of those fit a CU:
// 164 VGPRs, 43 KB of LDS; at the LoRA-step shape 512 work-groups took 58 us
// and 768 took 53). The buffer resource of a work-group's rows spans
// rows_per_block * cols * 2
// bytes, which stays at most 2^31: the offset that marks a column outside the
// matrix (2^31) must lie outside every range.
constexpr int64_t kMaxRangeBytes = (int64_t)1 << 31;

int64_t rows_per_block(int64_t rows, int64_t cols, bool three_per_cu) {
    const int64_t ncb = cols > 0 ? (cols + LR_TN - 1) / LR_TN : 1;
    int64_t nrb = ((three_per_cu ? 768 : 512) + ncb - 1) / ncb;
    const int64_t steps = (rows + LR_SM - 1) / LR_SM;
    if (nrb > steps) nrb = steps;
    if (nrb < 1) nrb = 1;
    int64_t per = (steps + nrb - 1) / nrb;
    int64_t max_per = cols > 0 ? kMaxRangeBytes / (cols * 2 * LR_SM) : per;
    if (max_per < 1) max_per = 1;  // callers reject such widths (check_common) before launching
    if (per > max_per) per = max_per;
    return per * LR_SM;
}

struct LoraPlan {
    int64_t ncb, nrb, rpb;
    int64_t row_bytes, col_bytes;  // partial buffers (ROW, COL)
};

LoraPlan plan(int64_t rows, int64_t cols, int R, bool row, bool col) {
    LoraPlan p;
    const int rp = rank_padded(R);
    p.ncb = (cols + LR_TN - 1) / LR_TN;
    p.rpb = rows_per_block(rows, cols, row && col && rp == 16);
    p.nrb = rows > 0 ? (rows + p.rpb - 1) / p.rpb : 0;
    p.row_bytes = row ? p.ncb * rows * rp * 4 : 0;
    p.col_bytes = col ? p.nrb * cols * rp * 4 : 0;
    return p;
}

unsigned reduce_grid(int64_t items, int R) {
    const int64_t v = items * (R / 4);
    return (unsigned)((v + 63) / 64);
}

template <typename Tr, int RP>
void launch_pass_t(const LoraArgs& a, bool row, bool col, dim3 grid, hipStream_t st) {
    if (row && col)
        hipLaunchKernelGGL((k_lora_pass<Tr, RP, true, true>), grid, dim3(256), 0, st, a);
    else if (row)
        hipLaunchKernelGGL((k_lora_pass<Tr, RP, true, false>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((k_lora_pass<Tr, RP, false, true>), grid, dim3(256), 0, st, a);
}

void launch_pass(const LoraArgs& a, int dtype, bool row, bool col, dim3 grid, hipStream_t st) {
    const int rp = rank_padded(a.rank);
    if (dtype == STM_BF16) {
        if (rp == 16) launch_pass_t<BF16, 16>(a, row, col, grid, st);
        else launch_pass_t<BF16, 32>(a, row, col, grid, st);
    } else {
        if (rp == 16) launch_pass_t<F16, 16>(a, row, col, grid, st);
        else launch_pass_t<F16, 32>(a, row, col, grid, st);
    }
}

RedJob red_job(const float* part, int blocks, int64_t items, int R, float scale, void* out) {
    return RedJob{part, blocks, items, scale, (uint16_t*)out, reduce_grid(items, R)};
}

// One launch for j0 and, when j1.grid > 0, j1 (both the same orientation).
void launch_reduce(const RedJob& j0, const RedJob& j1, int R, bool tr, int dtype, hipStream_t st) {
    const int rp = rank_padded(R);
    const unsigned grid = j0.grid + j1.grid;
    if (grid == 0) return;
    if (dtype == STM_BF16) {
        if (tr) hipLaunchKernelGGL((k_lora_reduce<BF16, true>), dim3(grid), dim3(256), 0, st, j0, j1, R, rp);
        else hipLaunchKernelGGL((k_lora_reduce<BF16, false>), dim3(grid), dim3(256), 0, st, j0, j1, R, rp);
    } else {
        if (tr) hipLaunchKernelGGL((k_lora_reduce<F16, true>), dim3(grid), dim3(256), 0, st, j0, j1, R, rp);
        else hipLaunchKernelGGL((k_lora_reduce<F16, false>), dim3(grid), dim3(256), 0, st, j0, j1, R, rp);
    }
}

void launch_reduce(const float* part, int blocks, int64_t items, int R, float scale, void* out, bool tr, int dtype,
                   hipStream_t st) {
    launch_reduce(red_job(part, blocks, items, R, scale, out), RedJob{}, R, tr, dtype, st);
}

int check_common(const char* what, int64_t rows, int64_t cols, int R, int dtype) {
    if (rows < 0 || cols < 0) return set_error(STM_ERR_INVALID, "%s: negative size", what);
    if (dtype != STM_BF16 && dtype != STM_F16) return set_error(STM_ERR_INVALID, "%s: dtype must be bf16 or fp16", what);
    if (R < 8 || R > 32 || R % 8) return set_error(STM_ERR_UNSUPPORTED, "%s: rank %d (needs 8, 16, 24 or 32)", what, R);
    if (cols % 8) return set_error(STM_ERR_UNSUPPORTED, "%s: %lld columns (needs a multiple of 8)", what, (long long)cols);
    // 256 rows of the large operand (a block's range plus the prefetch past it
    // stays below 2^32) and the ROW partials of one column block (one buffer
    // range) within kMaxRangeBytes
    if (cols * 2 * 4 * LR_SM > kMaxRangeBytes || rows * 32 * 4 > kMaxRangeBytes)
        return set_error(STM_ERR_UNSUPPORTED, "%s: %lld x %lld is too large", what, (long long)rows, (long long)cols);
    return STM_OK;
}

int check_ptrs(const char* what, std::initializer_list<const void*> ps) {
    for (const void* p : ps) {
        if (!p) return set_error(STM_ERR_INVALID, "%s: null pointer", what);
        if (!aligned(p, 16)) return set_error(STM_ERR_INVALID, "%s: operand not 16-byte aligned", what);
    }
    return STM_OK;
}

int check_workspace(const char* what, const void* ws, int64_t ws_bytes, int64_t need) {
    if (need == 0) return STM_OK;
    if (!ws || ws_bytes < need)
        return set_error(STM_ERR_INVALID, "%s: workspace of %lld bytes, needs %lld", what, (long long)ws_bytes,
                         (long long)need);
    if (!aligned(ws, 16)) return set_error(STM_ERR_INVALID, "%s: workspace not 16-byte aligned", what);
    return STM_OK;
}

}  // namespace
}  // namespace stm

using namespace stm;

extern "C" int64_t stm_lora_workspace_bytes(int64_t rows, int64_t cols, int rank, int op) {
    if (op < 0 || op > 2) return set_error(STM_ERR_INVALID, "lora_workspace_bytes: op %d (needs 0, 1 or 2)", op);
    // the shape limits of the entry points the workspace is for
    const int rc = check_common("lora_workspace_bytes", rows, cols, rank, STM_BF16);
    if (rc) return rc;
    const LoraPlan p = plan(rows, cols, rank, op != 2, op != 0);
    return p.row_bytes + p.col_bytes;
}

extern "C" int stm_lora_down(const void* X, const void* A, void* T, int64_t M, int64_t K, int rank, float scaling,
                             int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
    int rc = check_common("lora_down", M, K, rank, dtype);
    if (rc) return rc;
    if (M == 0) return STM_OK;
    if ((rc = check_ptrs("lora_down", {T}))) return rc;
    if (K > 0 && (rc = check_ptrs("lora_down", {X, A}))) return rc;
    const LoraPlan p = plan(M, K, rank, true, false);
    if ((rc = check_workspace("lora_down", workspace, workspace_bytes, p.row_bytes))) return rc;
    hipStream_t st = (hipStream_t)stream;
    float* part = (float*)workspace;
    if (K == 0) {
        // no reduction: T = 0 (the reduce sums zero blocks)
        launch_reduce(part, 0, M, rank, 0.f, T, false, dtype, st);
        return check_launch("lora_down");
    }
    if (M <= kDownRowsMax) {  // decode sizes: one launch, the workspace unused
        if (dtype == STM_BF16)
            launch_down_rows<BF16>(X, A, T, M, K, rank, scaling, st);
        else
            launch_down_rows<F16>(X, A, T, M, K, rank, scaling, st);
        return check_launch("lora_down");
    }
    LoraArgs a{(const uint16_t*)X, (const uint16_t*)A, nullptr, part, nullptr, M, K, rank, 1, (int)p.rpb};
    launch_pass(a, dtype, true, false, dim3((unsigned)p.ncb, (unsigned)p.nrb), st);
    launch_reduce(part, (int)p.ncb, M, rank, scaling, T, false, dtype, st);
    return check_launch("lora_down");
}

extern "C" int stm_lora_dy(const void* dY, const void* B, const void* T, void* U, void* dB, int64_t M, int64_t N,
                           int rank, float scaling, int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
    int rc = check_common("lora_dy", M, N, rank, dtype);
    if (rc) return rc;
    const bool col = dB != nullptr;
    if (M > 0 && (rc = check_ptrs("lora_dy", {U}))) return rc;
    if (col && N > 0 && (rc = check_ptrs("lora_dy", {dB}))) return rc;
    if (M > 0 && N > 0 && (rc = check_ptrs("lora_dy", {dY, B}))) return rc;
    if (col && M > 0 && N > 0 && (rc = check_ptrs("lora_dy", {T}))) return rc;
    const LoraPlan p = plan(M, N, rank, true, col);
    if ((rc = check_workspace("lora_dy", workspace, workspace_bytes, p.row_bytes + p.col_bytes))) return rc;
    hipStream_t st = (hipStream_t)stream;
    float* prow = (float*)workspace;
    float* pcol = (float*)((char*)workspace + p.row_bytes);
    if (M == 0 || N == 0) {
        if (M > 0) launch_reduce(prow, 0, M, rank, 0.f, U, false, dtype, st);
        if (col && N > 0) launch_reduce(pcol, 0, N, rank, 0.f, dB, false, dtype, st);
        return check_launch("lora_dy");
    }
    LoraArgs a{(const uint16_t*)dY, (const uint16_t*)B, (const uint16_t*)T, prow, pcol, M, N, rank, 0, (int)p.rpb};
    launch_pass(a, dtype, true, col, dim3((unsigned)p.ncb, (unsigned)p.nrb), st);
    // U and dB in one reduce launch
    launch_reduce(red_job(prow, (int)p.ncb, M, rank, scaling, U),
                  col ? red_job(pcol, (int)p.nrb, N, rank, 1.f, dB) : RedJob{}, rank, false, dtype, st);
    return check_launch("lora_dy");
}

extern "C" int stm_lora_da(const void* U, const void* X, void* dA, int64_t M, int64_t K, int rank, int dtype,
                           void* workspace, int64_t workspace_bytes, void* stream) {
    int rc = check_common("lora_da", M, K, rank, dtype);
    if (rc) return rc;
    if (K == 0) return STM_OK;
    if ((rc = check_ptrs("lora_da", {dA}))) return rc;
    if (M > 0 && (rc = check_ptrs("lora_da", {U, X}))) return rc;
    const LoraPlan p = plan(M, K, rank, false, true);
    if ((rc = check_workspace("lora_da", workspace, workspace_bytes, p.col_bytes))) return rc;
    hipStream_t st = (hipStream_t)stream;
    float* part = (float*)workspace;
    if (M == 0) {
        launch_reduce(part, 0, K, rank, 0.f, dA, true, dtype, st);
        return check_launch("lora_da");
    }
    LoraArgs a{(const uint16_t*)X, nullptr, (const uint16_t*)U, nullptr, part, M, K, rank, 0, (int)p.rpb};
    launch_pass(a, dtype, false, true, dim3((unsigned)p.ncb, (unsigned)p.nrb), st);
    launch_reduce(part, (int)p.nrb, K, rank, 1.f, dA, true, dtype, st);
    return check_launch("lora_da");
}
