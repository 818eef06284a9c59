// Fused NF4 dequant-GEMMs for gfx950 (bf16 / fp16 MFMA, fp32 accumulate).
//
// forward  Y[M, N]  = X[M, K] . W[N, K]^T  (+ bias) (+ T . L^T)
// backward dX[M, K] = dY[M, N] . W[N, K]            (+ U . At^T)
//
// Work-group tile BM x BN (activation rows x output columns), WM x WN waves,
// each wave (BM/WM) x (BN/WN) as a grid of v_mfma_f32_32x32x16 tiles; the
// reduction advances 64 per step (one NF4 block when blocksize = 64).
//
// Per step and LDS buffer:
//  * the activation tile (BM rows x 64) is copied global -> LDS with
//    global_load_lds_dwordx4 (no VGPR round trip): lane l of a wave writes the
//    16-byte LDS slot l of a 1 KB run, so the bank swizzle below is applied on the
//    global-address side (each lane fetches the chunk that belongs in its slot);
//  * the packed weight tile is loaded to VGPRs and dequantized with a 256-entry
//    (level_hi, level_lo) table in LDS, one fp32 product with the block absmax and
//    one round-to-nearest-even conversion -- the values the dequantize kernel
//    writes -- straight into LDS. Forward stores W rows [n][k]; backward stores
//    the transpose [k][n] (an 8 x 8 register transpose per thread) so that the
//    MFMA operand (8 consecutive reduction indices per lane) is one 16-byte read.
// LDS rows are 64 halfs = eight 16-byte chunks; chunk c of row r sits at
// c ^ ((r >> 1) & 7), so the 16 lanes of one 16-byte LDS pass (16 consecutive
// rows, one logical chunk) land on 16 different 16-byte bank groups.
// Two buffers: the loads of step k+1 are in flight while step k's MFMAs run.
//
// The MFMA computes the transposed tile (W-side operand as A, activation as B),
// so each lane's accumulators hold 4 consecutive output columns of one row and
// the epilogue writes 8-byte runs.
//
// MFMA layout (v_mfma_f32_32x32x16): lane l supplies A[l % 32][k-group l / 32]
// and B[k-group l / 32][l % 32] (8 halfs each; any k order common to A and B
// gives the same product); result v of lane l is C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32].
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "nf4_kernels.h"

// Tile shapes (measured best on MI355X at M = 8192, N = 14336, K = 4096):
// forward 256 x 256 with 8 waves (4 x 2), input gradient 256 x 256 with 4 waves.
#ifndef STM_FWD_BM
#define STM_FWD_BM 256
#define STM_FWD_BN 256
#define STM_FWD_WM 4
#define STM_FWD_WN 2
#endif
#ifndef STM_BWD_BM
#define STM_BWD_BM 256
#define STM_BWD_BN 256
#define STM_BWD_WM 2
#define STM_BWD_WN 2
#endif
#ifndef STM_GROUP_M
#define STM_GROUP_M 4
#endif

namespace stm {

namespace {

constexpr int BK = 64;  // reduction step

template <typename Tr>
__device__ __forceinline__ f32x16_t mfma(const uint4& a, const uint4& b, const f32x16_t& c) {
    if constexpr (Tr::tag == STM_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                      0, 0, 0);
}

template <typename Tr>
__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, const f32x4_t& c) {
    if constexpr (Tr::tag == STM_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                      0, 0, 0);
}

#ifndef STM_SWZ
#define STM_SWZ 1
#endif
__device__ __forceinline__ int swz_key(int row) { return STM_SWZ ? ((row >> 1) & 7) : (row & 7); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * 8 + (chunk ^ swz_key(row)); }

typedef __attribute__((address_space(3))) uint4 lds_uint4;
typedef int v2i32_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds_offset(const uint4* p) {
    return (uint32_t)(size_t)((const lds_uint4*)(p));
}

// 16 bytes global -> LDS for every lane of the wave; the LDS destination is
// lds_base + 16 * lane (lds_base wave-uniform, in M0). Issued as inline asm so
// the compiler does not treat every later LDS read as dependent on it (it
// cannot tell the two LDS buffers apart and would wait for the copy before the
// MFMA operand reads of the other buffer); completion is awaited explicitly
// with wait_vmem() before the barrier that publishes the buffer.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
    __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_base), "v"(src)
                     : "memory", "m0");
}
// 4 bytes global -> LDS for every lane; destination lds_base + 4 * lane.
__device__ __forceinline__ void dma4(const void* src, uint32_t lds_base) {
    __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds_base), "v"(src)
                     : "memory", "m0");
}
// The same copy from a wave-uniform 64-bit base plus a 32-bit per-lane byte offset
// (global_load_lds with an SGPR base: no 64-bit address arithmetic per copy).
__device__ __forceinline__ void dma16_s(const void* base, uint32_t voff, uint32_t lds_base) {
    const uint64_t b = (uint64_t)(size_t)base;
    const uint64_t sb = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const void* sbase = (const void*)(size_t)sb;
    __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_base), "v"(voff), "s"(sbase)
                     : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(0) (expcnt, lgkmcnt left at their maxima). Emitted through the
// builtin so the compiler's own wait-count bookkeeping sees it and inserts no
// further waits for the weight registers loaded before it.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Expert e owns rows [row0, row0 + rows) of the activations/outputs and the
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

// Tile order: work-groups are dispatched round-robin over the 8 XCDs, so ids
// i, i + 8, i + 16, ... share an L2. Give each XCD a contiguous run of tiles and
// walk them GROUP_M activation tiles at a time so concurrently running tiles on
// one XCD reuse the same activation rows and weight rows. With 32 CUs per XCD,
// GROUP_M = 4 runs 4 activation x 8 weight tiles together; measured at
// M = 8192 on W [14336, 4096] it fetches 735 MB per forward from beyond L2
// (GROUP_M = 8: 1072 MB, 2: 820 MB) and is 1-4 % faster.
__device__ __forceinline__ void tile_coords(int64_t pid, int64_t ntm, int64_t ntn, int64_t& tm, int64_t& tn,
                                            bool xcd_runs = true) {
    const int64_t T = ntm * ntn;
    const int64_t T8 = (T / 8) * 8;
    if (xcd_runs && pid < T8) pid = (pid % 8) * (T / 8) + pid / 8;
    const int64_t per_group = (int64_t)STM_GROUP_M * ntn;
    const int64_t grp = pid / per_group;
    const int64_t first = grp * STM_GROUP_M;
    const int64_t gsize = (ntm - first) < STM_GROUP_M ? (ntm - first) : STM_GROUP_M;
    const int64_t in = pid % per_group;
    tm = first + in % gsize;
    tn = in / gsize;
}

// Grouped launches (experts): item w of a work-group runs on XCD w % 8, so the
// item list (expert-major: an expert's tiles are consecutive) is cut into 8
// contiguous runs, one per XCD. An expert's tiles then run together on one XCD
// and share its rows of the activations (and the expert's weight) in that
// XCD's L2, instead of being spread over all eight. Dense launches keep the
// per-tile order of tile_coords. A bijection on [0, work).
__device__ __forceinline__ int64_t item_order(int64_t w, int64_t work, int num_groups) {
    if (num_groups <= 1) return w;
    const int64_t W8 = (work / 8) * 8;
    return w < W8 ? (w % 8) * (work / 8) + w / 8 : w;
}

// 1: grouped launches of the register-weight kernels walk a compact item list
// (GroupedPlan); 0: every expert gets ceil(max_rows / BM) row-tile slots.
#ifndef STM_GROUPED_PLAN
#define STM_GROUPED_PLAN 1
#endif

// Compact item list of a grouped launch, built by every work-group from the
// device offsets at kernel start. Expert e holds nt_e = ceil(rows_e / BM) row
// tiles. Its last tile is a tail when it holds at most 128 rows (a short item:
// a quarter or half of the MFMAs, the full weight work); every other tile is a
// main tile. Items run all main tiles first (experts in order, an expert's
// tiles column-tile-major, as the slot order had them), then all tails, each
// class in contiguous per-XCD runs. So every work-group gets the same number
// of main items (up to one), the cheap tails even out the rest, and slots past
// an expert's rows are never enumerated. Thread t owns experts 2t and 2t + 1.
constexpr int kPlanExperts = 512;
struct GroupedPlan {
    int off[kPlanExperts + 1];       // the expert offsets
    int pre_main[kPlanExperts + 1];  // exclusive prefix of main tiles over experts
    int pre_tail[kPlanExperts + 1];  // exclusive prefix of tails (0 or 1 per expert)
};

__device__ __forceinline__ bool plan_usable(const GemmArgs& g) {
    return STM_GROUPED_PLAN && g.num_groups > 1 && g.offsets && g.num_groups <= kPlanExperts && g.splits == 1;
}

// Ends with a barrier: the plan is visible to every wave.
template <int BM>
__device__ void build_plan(const GemmArgs& g, GroupedPlan& P, int tid) {
    static_assert(2 * 256 == kPlanExperts, "256 threads, two experts each");
    __shared__ int wave_tot[2][4];
    const int E = g.num_groups, lane = tid & 63, wave = tid >> 6;
    int m[2], t[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int e = 2 * tid + i;
        m[i] = t[i] = 0;
        if (e < E) {
            const int r0 = g.offsets[e], r1 = g.offsets[e + 1];
            P.off[e] = r0;
            if (e == E - 1) P.off[E] = r1;
            const int rows = r1 - r0;
            const int nt = (rows + BM - 1) / BM;
            t[i] = nt > 0 && rows - (nt - 1) * BM <= 128 ? 1 : 0;
            m[i] = nt - t[i];
        }
    }
    int sm = m[0] + m[1], st = t[0] + t[1];  // inclusive scans over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int om = __shfl_up(sm, d), ot = __shfl_up(st, d);
        if (lane >= d) sm += om, st += ot;
    }
    if (lane == 63) wave_tot[0][wave] = sm, wave_tot[1][wave] = st;
    __syncthreads();
    for (int v = 0; v < wave; ++v) sm += wave_tot[0][v], st += wave_tot[1][v];
    const int em = sm - m[0] - m[1], et = st - t[0] - t[1];  // exclusive
    P.pre_main[2 * tid] = em;
    P.pre_main[2 * tid + 1] = em + m[0];
    P.pre_tail[2 * tid] = et;
    P.pre_tail[2 * tid + 1] = et + t[0];
    if (tid == 255) P.pre_main[kPlanExperts] = sm, P.pre_tail[kPlanExperts] = st;
    __syncthreads();
}

// Item w of the plan's list: expert e, row tile tm, column tile tn (ntn column
// tiles). Every lane of the wave takes part (the expert search is a ballot).
template <int BM>
__device__ __forceinline__ void plan_item(const GroupedPlan& P, int E, int64_t ntn, int64_t w, int64_t main_work,
                                          int64_t work, int lane, int& e, int64_t& tm, int64_t& tn) {
    const bool is_main = w < main_work;
    int64_t u = is_main ? w : w - main_work;
    u = item_order(u, is_main ? main_work : work - main_work, 2);
    const int* pre = is_main ? P.pre_main : P.pre_tail;
    // the expert: one less than the number of experts whose first item is at or before u
    int cnt = 0;
    for (int j = 0; 64 * j < E; ++j) {
        const int ee = 64 * j + lane;
        cnt += __popcll(__ballot(ee < E && (int64_t)pre[ee] * ntn <= u));
    }
    e = __builtin_amdgcn_readfirstlane(cnt - 1);
    const int64_t local = u - (int64_t)pre[e] * ntn;
    if (is_main) {
        const int64_t n_e = pre[e + 1] - pre[e];
        tn = local / n_e;
        tm = local % n_e;
    } else {
        const int rows = P.off[e + 1] - P.off[e];
        tm = (rows + BM - 1) / BM - 1;
        tn = local;
    }
}

__device__ __forceinline__ Group plan_group(const GemmArgs& g, const GroupedPlan& P, int e) {
    Group r;
    r.row0 = P.off[e];
    r.rows = (int64_t)P.off[e + 1] - r.row0;
    const int64_t wnum = g.N * g.K;
    r.packed = g.packed + (int64_t)e * (wnum / 2);
    r.absmax = g.absmax + (int64_t)e * (wnum / g.blocksize);
    return r;
}

// Activation staging: the tile rows [m0, m0 + BM) x [k0, k0 + 64) are copied
// into an LDS buffer (BM x 8 chunks) with XI direct copies per wave per step.
// Per-lane global row pointers and the wave-uniform LDS bases of both buffers
// are computed once; a step only adds k0. Rows past the valid range re-read the
// last valid row: they only feed output rows that are never stored.
template <int BM, int NW>
struct ActStage {
    static constexpr int XI = BM / (8 * NW);
    const uint16_t* src[XI];
    uint32_t lds[2][XI];

    __device__ __forceinline__ void init(const uint16_t* base, int64_t ld, int64_t m0, int64_t rows, const uint4* buf0,
                                         const uint4* buf1, int wave, int lane) {
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int r0 = (wave * XI + i) * 8;
            const int r = r0 + (lane >> 3);
            const int c = (lane & 7) ^ swz_key(r);
            int64_t row = m0 + r;
            row = row < rows ? row : rows - 1;
            src[i] = base + row * ld + c * 8;
            lds[0][i] = __builtin_amdgcn_readfirstlane(lds_offset(buf0 + r0 * 8));
            lds[1][i] = __builtin_amdgcn_readfirstlane(lds_offset(buf1 + r0 * 8));
        }
    }
    __device__ __forceinline__ void issue(int64_t k0, int buf) const {
#pragma unroll
        for (int i = 0; i < XI; ++i) dma16(src[i] + k0, lds[buf][i]);
    }
};

// ActStage with a wave-uniform base and 32-bit byte offsets (the tile's rows
// must lie within 4 GiB of the base).
template <int BM, int NW>
struct ActStageS {
    static constexpr int XI = BM / (8 * NW);
    const uint16_t* base;
    uint32_t off[XI];
    uint32_t lds[2][XI];

    __device__ __forceinline__ void init(const uint16_t* b, int64_t ld, int64_t m0, int64_t rows, const uint4* buf0,
                                         const uint4* buf1, int wave, int lane) {
        base = b;
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int r0 = (wave * XI + i) * 8;
            const int r = r0 + (lane >> 3);
            const int c = (lane & 7) ^ swz_key(r);
            int64_t row = m0 + r;
            row = row < rows ? row : rows - 1;
            off[i] = (uint32_t)((row * ld + c * 8) * 2);
            lds[0][i] = __builtin_amdgcn_readfirstlane(lds_offset(buf0 + r0 * 8));
            lds[1][i] = __builtin_amdgcn_readfirstlane(lds_offset(buf1 + r0 * 8));
        }
    }
    __device__ __forceinline__ void issue(int64_t k0, int buf) const {
#pragma unroll
        for (int i = 0; i < XI; ++i) dma16_s(base + k0, off[i], lds[buf][i]);
    }
};

// Level table: entry (byte b, copy c) = (level[b >> 4], level[b & 15]) at
// index 16 b + c. Lane l reads copy l % 16, so the 16 lanes of one LDS pass of
// a 64-bit read always hit 16 different bank pairs (a single shared copy makes
// random byte values collide on banks several times per read).
constexpr int LUT_COPIES = 16;

// Level i (0..15) of the codebook from immediates: no memory access.
__device__ __forceinline__ float level_from_immediates(int i) {
    float v = kLevelsDev[0];
#pragma unroll
    for (int k = 1; k < 16; ++k) v = i == k ? kLevelsDev[k] : v;
    return v;
}

// Entries (level[b >> 4], level[b & 15]) at index copies * b + c, written by NT
// threads. Pair p = (lo, c) = (p / copies, p % copies) belongs to thread
// p % NT; it writes the 16 entries b = 16 hi + lo, hi = 0..15, whose first
// level is an immediate and whose second is the thread's one selected level:
// 16 independent LDS writes, no memory or cross-lane round trips.
template <int NT, int COPIES>
__device__ __forceinline__ void fill_level_table(float2* lut, int tid) {
    constexpr int PAIRS = 16 * COPIES, ITERS = (PAIRS + NT - 1) / NT;
#pragma unroll
    for (int i = 0; i < ITERS; ++i) {
        const int p = tid + NT * i;
        if (PAIRS % NT != 0 && p >= PAIRS) break;
        const int lo = p / COPIES, c = p % COPIES;
        const float lv = level_from_immediates(lo);
#pragma unroll
        for (int hi = 0; hi < 16; ++hi) lut[(16 * hi + lo) * COPIES + c] = make_float2(kLevelsDev[hi], lv);
    }
}

template <int NT>
__device__ __forceinline__ void fill_lut(float2* lut, int tid) {
    fill_level_table<NT, LUT_COPIES>(lut, tid);
}

template <int FA, int FB>
__device__ __forceinline__ void zero_acc(f32x16_t (&acc)[FA][FB]) {
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
}

// Rank-R term: acc[i][j] += Wside[rows] . Xside[cols]^T, both row-major with R contiguous.
// Accumulator row r of fragment i is weight-side row wrow_base + 32 i + (r ^ CX).
template <typename Tr, int FA, int FB, int CX = 0>
__device__ __forceinline__ void lora_term(f32x16_t (&acc)[FA][FB], const uint16_t* __restrict__ wside,
                                          int64_t wrow_base, int64_t wrows, const uint16_t* __restrict__ xside,
                                          int64_t xrow_base, int64_t xrows, int R, int lane) {
    for (int r0 = 0; r0 < R; r0 += 16) {
        uint4 a[FA], b[FB];
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            int64_t row = wrow_base + i * 32 + ((lane & 31) ^ CX);
            row = row < wrows ? row : wrows - 1;
            a[i] = *reinterpret_cast<const uint4*>(wside + row * R + r0 + 8 * (lane >> 5));
        }
#pragma unroll
        for (int j = 0; j < FB; ++j) {
            int64_t row = xrow_base + j * 32 + (lane & 31);
            row = row < xrows ? row : xrows - 1;
            b[j] = *reinterpret_cast<const uint4*>(xside + row * R + r0 + 8 * (lane >> 5));
        }
#pragma unroll
        for (int i = 0; i < FA; ++i)
#pragma unroll
            for (int j = 0; j < FB; ++j) acc[i][j] = mfma<Tr>(a[i], b[j], acc[i][j]);
    }
}

// acc[i][j] holds C^T: rows = output columns (wcol_base + i*32 + ...), cols = output rows.
template <typename Tr, int FA, int FB>
__device__ __forceinline__ void store_tile(const f32x16_t (&acc)[FA][FB], uint16_t* __restrict__ out, int64_t ld,
                                           int64_t ocol_base, int64_t ocols, int64_t orow_base, int64_t orows,
                                           const uint16_t* __restrict__ bias, int lane) {
#pragma unroll
    for (int j = 0; j < FB; ++j) {
        const int64_t orow = orow_base + j * 32 + (lane & 31);
        if (orow >= orows) continue;
        uint16_t* dst = out + orow * ld;
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            f32x16_t a = acc[i][j];
            if constexpr (FA * FB >= 8) __asm__ volatile("" : "+v"(a));  // one fragment at a time out of 128+ accumulators
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t col = ocol_base + i * 32 + 8 * q + 4 * (lane >> 5);
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = a[4 * q + e];
                    if (bias && col + e < ocols) v[e] += Tr::to_f32(bias[col + e]);
                }
                if (col + 3 < ocols) {
                    uint2 pk;
                    pk.x = Tr::pack2(v[0], v[1]);
                    pk.y = Tr::pack2(v[2], v[3]);
                    *reinterpret_cast<uint2*>(dst + col) = pk;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < ocols) dst[col + e] = Tr::from_f32(v[e]);
                }
            }
        }
    }
}

// fp32 partial tile of one split: the same element mapping as store_tile,
// 16-byte runs (4 consecutive output columns per lane).
template <int FA, int FB>
__device__ __forceinline__ void store_tile_f32(const f32x16_t (&acc)[FA][FB], float* __restrict__ out, int64_t ld,
                                               int64_t ocol_base, int64_t ocols, int64_t orow_base, int64_t orows,
                                               int lane) {
#pragma unroll
    for (int j = 0; j < FB; ++j) {
        const int64_t orow = orow_base + j * 32 + (lane & 31);
        if (orow >= orows) continue;
        float* dst = out + orow * ld;
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            f32x16_t a = acc[i][j];
            if constexpr (FA * FB >= 8) __asm__ volatile("" : "+v"(a));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t col = ocol_base + i * 32 + 8 * q + 4 * (lane >> 5);
                if (col + 3 < ocols) {
                    *reinterpret_cast<float4*>(dst + col) = make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < ocols) dst[col + e] = a[4 * q + e];
                }
            }
        }
    }
}

#ifndef STM_RW_LDS_STORE
#define STM_RW_LDS_STORE 1
#endif
// Output tile through LDS: each wave writes its slice (32 FA columns x 32 FB
// rows, NP passes of 32 FB / NP rows) into a private LDS stage (rows of CH =
// 4 FA chunks of 16 bytes, chunk slot c ^ (row % CH)), then stores it with
// 16-byte lanes, CH lanes per output row, so every store instruction writes
// whole cache lines. Direct stores from the accumulator layout write 8 bytes
// per lane across 32 rows and cost about a tenth of a 64-step 256 x 256 tile.
// The caller has made the stage free (barrier) and frees it for others after
// (barrier). ocols % 8 == 0. CX = 1: accumulator row r holds column r ^ 1.
template <typename Tr, int FA, int FB, int CX = 0, int NP = 2>
__device__ __forceinline__ void store_tile_lds(const f32x16_t (&acc)[FA][FB], uint16_t* __restrict__ out, int ld,
                                               int ocol_base, int ocols, int orow_base, int orows,
                                               const uint16_t* __restrict__ bias, int lane, uint4* stage,
                                               bool nt = false) {
    static_assert(FB % NP == 0 && (FA == 1 || FA == 2 || FA == 4), "32, 64 or 128 columns per wave");
    // (the register-weight kernels use FA = 2, NP = 2; the LDS-weight kernels'
    // 128 x 128 tiles store a quarter of the bytes per item and measured no gain)
    constexpr int FP = FB / NP, RP = 32 * FP, CH = 4 * FA, RPI = 64 / CH;  // rows per pass / per store
    const int hi = lane >> 5, c0 = ocol_base + 4 * hi;
    float bv[FA][4][4];
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int col = c0 + i * 32 + 8 * q + (e ^ CX);
                bv[i][q][e] = (bias && col < ocols) ? Tr::to_f32(bias[col]) : 0.0f;
            }
    uint8_t* st = reinterpret_cast<uint8_t*>(stage);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        if (orow_base + p * RP >= orows) break;  // no valid row left (uniform: the wave's base)
#pragma unroll
        for (int jj = 0; jj < FP; ++jj) {
            const int rr = 32 * jj + (lane & 31);
#pragma unroll
            for (int i = 0; i < FA; ++i) {
                f32x16_t a = acc[i][p * FP + jj];
                __asm__ volatile("" : "+v"(a));
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = a[4 * q + e] + bv[i][q][e];
                    uint2 pk;
                    pk.x = CX ? Tr::pack2(v[1], v[0]) : Tr::pack2(v[0], v[1]);
                    pk.y = CX ? Tr::pack2(v[3], v[2]) : Tr::pack2(v[2], v[3]);
                    const int slot = (4 * i + q) ^ (rr & (CH - 1));
                    *reinterpret_cast<uint2*>(st + rr * (16 * CH) + slot * 16 + 8 * hi) = pk;
                }
            }
        }
        // 16-byte lanes: row rr = RPI it + lane / CH, chunk lane % CH
#pragma unroll
        for (int it = 0; it < RP / RPI; ++it) {
            const int rr = RPI * it + lane / CH, c = lane % CH;
            const uint4 v = stage[rr * CH + (c ^ (rr & (CH - 1)))];
            const int orow = orow_base + p * RP + rr, col = ocol_base + 8 * c;
            if (orow < orows && col < ocols) {
                if (nt)
                    __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v),
                                                reinterpret_cast<u32x4_t*>(out + (orow * ld + col)));
                else
                    *reinterpret_cast<uint4*>(out + (orow * ld + col)) = v;
            }
        }
    }
}

// Step range of split z of `steps` reduction steps.
__device__ __forceinline__ void split_range(int steps, int splits, int z, int& begin, int& count) {
    begin = (int)(((int64_t)z * steps) / splits);
    count = (int)(((int64_t)(z + 1) * steps) / splits) - begin;
}

// One 16-deep MFMA sub-step kk of a 64-deep step.
template <typename Tr, int FA, int FB>
__device__ __forceinline__ void mma_kk(f32x16_t (&acc)[FA][FB], const uint4* sw, int wrow0, const uint4* sx,
                                       int xrow0, int lane, int kk) {
    const int ch = kk * 2 + (lane >> 5);
    uint4 a[FA], b[FB];
#pragma unroll
    for (int i = 0; i < FA; ++i) a[i] = sw[swz(wrow0 + i * 32 + (lane & 31), ch)];
#pragma unroll
    for (int j = 0; j < FB; ++j) b[j] = sx[swz(xrow0 + j * 32 + (lane & 31), ch)];
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j) acc[i][j] = mfma<Tr>(a[i], b[j], acc[i][j]);
}

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// An opaque copy of the lane index. Values computed from it stay after the point
// where it is taken: per-work-item lane offsets are recomputed per item, and
// epilogue addresses after the main loop, instead of being computed once up
// front and held (spilled) across the main loop.
__device__ __forceinline__ int opaque_lane(int lane) {
    __asm__ volatile("" : "+v"(lane));
    return lane;
}

// Shared main loop. Step s computes on buffers (s & 1) while the activation
// tile of step s + 1 streams into the other LDS buffer, the weight tile of
// step s + 1 (already in VGPRs) is dequantized into the other weight buffer,
// and the packed weight tile of step s + 2 is fetched into VGPRs.
//
// The dequantization is software-pipelined against the MFMAs: it is cut into
// four pieces; the level-table reads of piece i + 1 are issued before the
// MFMAs of sub-step i and its arithmetic and LDS writes follow them, so the
// VALU work and the LDS latency hide under the matrix pipe. Scheduling fences
// keep the compiler from regrouping the pieces.
//
// Prefetch indices clamp at the last step, so the loop body has no branches;
// the redundant copies at the end land in a buffer that is not read again.
template <typename Tr, int BM, int BN, int WM, int WN, int FW, int FX, typename WS>
__device__ __forceinline__ void run_pipeline(f32x16_t (&acc)[FW][FX], const uint16_t* act, int64_t ld, int64_t m0,
                                             int64_t rows, int KT, uint4* sA0, uint4* sA1, uint4* sB0, uint4* sB1,
                                             WS& ws, int wave, int lane) {
    constexpr int NW = WM * WN;
    const int wn = wave % WN, wm = wave / WN;
    const int wrow0 = wn * (BN / WN), xrow0 = wm * (BM / WM);
    typename WS::Regs w0, w1;
    ActStage<BM, NW> as;
    as.init(act, ld, m0, rows, sA0, sA1, wave, lane);

    as.issue(0, 0);
    ws.load(0, w0);
    __syncthreads();  // level table ready
    ws.store_all(w0, sB0);
    ws.load(KT > 1 ? 1 : 0, w1);
    wait_vmem();
    __syncthreads();

    auto step = [&](int s, const uint4* sAc, const uint4* sBc, int next_buf, uint4* sBn, typename WS::Regs& wcur,
                    typename WS::Regs& wnext) {
        const int s1 = s + 1 < KT ? s + 1 : KT - 1;
        const int s2 = s + 2 < KT ? s + 2 : KT - 1;
        as.issue((int64_t)s1 * BK, next_buf);
        ws.load(s2, wnext);
        typename WS::Pending pend[2];
        ws.issue(wcur, 0, pend[0]);
        sched_fence();
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            mma_kk<Tr, FW, FX>(acc, sBc, wrow0, sAc, xrow0, lane, kk);
            if (kk + 1 < BK / 16) ws.issue(wcur, kk + 1, pend[(kk + 1) & 1]);
            ws.finish(wcur, kk, pend[kk & 1], sBn);
            sched_fence();
        }
        ws.flush(sBn);
        wait_vmem();
        __syncthreads();
    };
    int s = 0;
    for (; s + 1 < KT; s += 2) {
        step(s, sA0, sB0, 1, sB1, w1, w0);
        step(s + 1, sA1, sB1, 0, sB0, w0, w1);
    }
    if (s < KT) {
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) mma_kk<Tr, FW, FX>(acc, sB0, wrow0, sA0, xrow0, lane, kk);
    }
}

// ------------------------------------------------------------------ forward
// Weight staging for the forward kernel: each thread owns WC 16-byte chunks
// of packed codes per step (row cidx / 2, 32-element half cidx % 2, cidx =
// tid + j * NT). Piece i of the dequantization is packed word i of every chunk
// (8 elements -> one 16-byte LDS chunk).
template <typename Tr, int WC, int NT>
struct FwdStage {
    struct Regs {
        uint4 q[WC];
        float a[WC];
    };
    struct Pending {
        float2 c[WC][4];
    };
    const uint8_t* wp[WC];
    const float* wa[WC];
    const float2* lut;
    int tid, bshift;
    int64_t kbase;  // first reduction index of this work-group's step range

    __device__ __forceinline__ void load(int s, Regs& w) const {
        const int64_t k0 = kbase + (int64_t)s * BK;
#pragma unroll
        for (int j = 0; j < WC; ++j) {
            w.q[j] = *reinterpret_cast<const uint4*>(wp[j] + k0 / 2);
            w.a[j] = wa[j][k0 >> bshift];
        }
    }
    __device__ __forceinline__ static uint32_t word(const uint4& q, int i) {
        return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
    }
    __device__ __forceinline__ void issue(const Regs& w, int i, Pending& p) const {
#pragma unroll
        for (int j = 0; j < WC; ++j) {
            const uint32_t x = word(w.q[j], i);
#pragma unroll
            for (int b = 0; b < 4; ++b) p.c[j][b] = lut[((x >> (8 * b)) & 0xFFu) * LUT_COPIES];
        }
    }
    __device__ __forceinline__ void finish(const Regs& w, int i, const Pending& p, uint4* dst) const {
#pragma unroll
        for (int j = 0; j < WC; ++j) {
            const int cidx = tid + j * NT;
            const float a = w.a[j];
            uint4 o;
            o.x = Tr::pack2(opaque(p.c[j][0].x * a), opaque(p.c[j][0].y * a));
            o.y = Tr::pack2(opaque(p.c[j][1].x * a), opaque(p.c[j][1].y * a));
            o.z = Tr::pack2(opaque(p.c[j][2].x * a), opaque(p.c[j][2].y * a));
            o.w = Tr::pack2(opaque(p.c[j][3].x * a), opaque(p.c[j][3].y * a));
            dst[swz(cidx >> 1, (cidx & 1) * 4 + i)] = o;
        }
    }
    __device__ __forceinline__ void flush(uint4*) const {}
    __device__ __forceinline__ void store_all(const Regs& w, uint4* dst) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            Pending p;
            issue(w, i, p);
            finish(w, i, p, dst);
        }
    }
};

template <typename Tr, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM* WN * 64) void k_gemm_fwd(GemmArgs g) {
    constexpr int NW = WM * WN, NT = NW * 64;
    constexpr int FX = BM / WM / 32;  // activation-side fragments per wave (MFMA B operand)
    constexpr int FW = BN / WN / 32;  // weight-side fragments per wave (MFMA A operand)
    constexpr int WC = BN * 2 / NT;   // 16-byte packed weight chunks per thread per step
    static_assert(BM % (8 * NW) == 0 && (BN * 2) % NT == 0, "tile / wave mismatch");
    __shared__ float2 lut_all[256 * LUT_COPIES];
    __shared__ uint4 sA0[BM * 8], sA1[BM * 8];
    __shared__ uint4 sB0[BN * 8], sB1[BN * 8];

    // (large tiles) the wave index as a uniform value: wave-derived offsets then
    // live in SGPRs instead of taking VGPRs from the accumulators' neighbours
    constexpr bool kLargeAcc = (BM / WM / 32) * (BN / WN / 32) >= 8;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = kLargeAcc ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    fill_lut<NT>(lut_all, tid);

    const int64_t K = g.K, N = g.N;
    const int64_t ntm = (g.M + BM - 1) / BM, ntn = (N + BN - 1) / BN, tiles = ntm * ntn;
    const int64_t work = tiles * g.num_groups * g.splits;
    // Work item w = (tile, group, split); a work-group takes items w, w + grid, ...
    // (one item each when the grid covers them all, else a persistent loop that
    // fills the level table once and overlaps one item's stores with the next
    // item's first loads).
    for (int64_t w = blockIdx.x; w < work; w += gridDim.x) {
    const int64_t wi = item_order(w, work, g.num_groups);
    const int64_t rest = wi / tiles;
    const int z = (int)(rest / g.num_groups);
    const Group grp = group_of(g, (int)(rest % g.num_groups));
    int64_t tm, tn;
    tile_coords(wi % tiles, ntm, ntn, tm, tn, g.num_groups == 1);
    const int64_t m0 = tm * BM, n0 = tn * BN;
    if (m0 >= grp.rows) continue;  // uniform over the work-group

    int s_begin, KT;
    split_range((int)(K / BK), g.splits, z, s_begin, KT);
    const uint16_t* __restrict__ X = reinterpret_cast<const uint16_t*>(g.a) + grp.row0 * K + (int64_t)s_begin * BK;
    const int64_t kblocks = K / g.blocksize;

    FwdStage<Tr, WC, NT> ws;
    ws.lut = lut_all + (lane & (LUT_COPIES - 1));
    ws.tid = tid;
    ws.bshift = ilog2(g.blocksize);
    ws.kbase = (int64_t)s_begin * BK;
#pragma unroll
    for (int j = 0; j < WC; ++j) {
        const int cidx = tid + j * NT;
        int64_t n = n0 + (cidx >> 1);
        n = n < N ? n : N - 1;  // rows past N only feed columns that are never stored
        ws.wp[j] = grp.packed + n * (K / 2) + (cidx & 1) * 16;
        ws.wa[j] = grp.absmax + n * kblocks;
    }

    f32x16_t acc[FW][FX];
    zero_acc(acc);
    run_pipeline<Tr, BM, BN, WM, WN, FW, FX>(acc, X, K, m0, grp.rows, KT, sA0, sA1, sB0, sB1, ws, wave, lane);

    const int64_t col_base = n0 + wn * (BN / WN), row_base = m0 + wm * (BM / WM);
    const int lane_e = FW * FX >= 8 ? opaque_lane(lane) : lane;
    if (g.lora_rank > 0 && z == 0)
        lora_term<Tr, FW, FX>(acc, reinterpret_cast<const uint16_t*>(g.lora_w), col_base, N,
                              reinterpret_cast<const uint16_t*>(g.lora_x) + grp.row0 * g.lora_rank, row_base,
                              grp.rows, g.lora_rank, lane_e);
    if (g.splits > 1)
        store_tile_f32<FW, FX>(acc, g.partial + (int64_t)z * g.M * N, N, col_base, N, row_base, grp.rows, lane_e);
    else
        store_tile<Tr, FW, FX>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * N, N, col_base, N, row_base,
                               grp.rows, reinterpret_cast<const uint16_t*>(g.bias), lane_e);
    __syncthreads();  // all waves are done with the LDS buffers before the next item fills them
    }
}

// ------------------------------------------------- forward, register weights
// Y tile BM x 256 with 4 WM waves; wave (wm, wn) owns the 64 output columns
// [n0 + 64 wn, n0 + 64 wn + 64) over rows [m0 + wm BM / WM, ...) (2 x BM/WM/32
// MFMA tiles; 256 accumulators per lane for BM = 256, WM = 1, the product
// configuration). Because no two waves along N share a weight column, each wave
// dequantizes its weight fragments straight into MFMA operand registers: the
// weight never goes through LDS, only the activation tile (shared by the waves)
// and the level table do. Runs the unsplit 256 x 256 forwards (single-matrix and
// grouped); it can also store a split's fp32 partial tile, but split forwards
// measured faster on the LDS-weight kernel (see rw_split_ok).
//
// Reduction order inside a 64-deep step: lane half h = lane / 32 of a weight row
// loads the 16 packed bytes of k in [32 h, 32 h + 32); MFMA sub-step j takes
// packed word j, i.e. k = 32 h + 8 j + (0..7). The activation operand of lane
// (row, h) at sub-step j is the 16-byte LDS chunk 4 h + j of its row -- the same
// k set, so the product is the plain dot product over the step.
//
// Step s (activation buffers alternate): copy the activation tile of step s + 1
// into the other LDS buffer and fetch the packed weights of step s + 2 into
// VGPRs; run sub-steps 0..2 on operands already in registers; wait for the
// copies, barrier; run sub-step 3, whose operands were read before the barrier,
// while the first activation fragments of step s + 1 are read. Each sub-step
// reloads every activation fragment in place right after its two MFMAs, and
// rewrites one weight-fragment slot just after the slot's MFMAs (the table reads
// for it issued one sub-step earlier), so neither operand is double-buffered
// (32 + 32 VGPRs for BM = 256). sched_group_barrier interleaves each
// sub-step as 2 VALU, 1 LDS read, 1 MFMA per slot; with one wave per SIMD, work
// that is not interleaved with MFMAs leaves the matrix core idle.

// Level table for the register-weight kernel: entry (byte b, copy c) at
// float2 index 32 b + c, so the LDS byte address of a lookup is
// (b << 8) | (8 c), one v_perm_b32 from the packed word and the lane's copy
// offset; lanes 0..31 of a pass read 32 different copies (all 64 banks).
constexpr int RW_LUT_COPIES = 32;

template <int NT>
__device__ __forceinline__ void fill_lut_rw(float2* lut, int tid) {
    fill_level_table<NT, RW_LUT_COPIES>(lut, tid);
}

template <typename Tr, int FA = 2>
struct RwWeights {
    struct Raw {
        uint4 q[FA];
        float a[FA];
    };
    const uint8_t* packed;  // the group's packed weight
    const float* absmax;    // the group's absmax
    uint32_t woff[FA];      // byte offset of this lane's 16-byte run of the first step, fragment i
    uint32_t aoff[FA];      // absmax index of the start of weight row (fragment i)
    int64_t kbase;          // first reduction index of the work item's step range
    int bshift;
    uint32_t lut_base;     // LDS byte address of the level table
    uint32_t copy_off;     // 8 * (lane % 32)

    __device__ __forceinline__ void load(int64_t k0, Raw& r) const {
        load_words(k0, r);
        load_absmax(k0, r);
    }
    __device__ __forceinline__ void load_words(int64_t k0, Raw& r) const {
#pragma unroll
        for (int i = 0; i < FA; ++i) r.q[i] = *reinterpret_cast<const uint4*>(packed + (woff[i] + (uint32_t)(k0 / 2)));
    }
    __device__ __forceinline__ void load_absmax(int64_t k0, Raw& r) const {
#pragma unroll
        for (int i = 0; i < FA; ++i) r.a[i] = absmax[aoff[i] + (uint32_t)((kbase + k0) >> bshift)];
    }
    __device__ __forceinline__ static uint32_t word(const uint4& q, int j) {
        return j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
    }
    // table reads for sub-step j of every fragment (4 lookups each)
    __device__ __forceinline__ void issue(const Raw& r, int j, f32x2_t (&p)[FA][4]) const {
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            const uint32_t x = word(r.q[i], j);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                // bytes: [0] = copy offset, [1] = packed byte b of x, [2], [3] = 0
                const uint32_t addr = __builtin_amdgcn_perm(copy_off, x, 0x0C0C0004u | ((uint32_t)b << 8));
                p[i][b] = *(const __attribute__((address_space(3))) f32x2_t*)(size_t)(lut_base + addr);
            }
        }
    }
    __device__ __forceinline__ static void finish(const Raw& r, const f32x2_t (&p)[FA][4], uint4 (&out)[FA]) {
        finish_a(r.a, p, out);
    }
    __device__ __forceinline__ static void finish_a(const float (&am)[FA], const f32x2_t (&p)[FA][4],
                                                    uint4 (&out)[FA]) {
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            const float a = am[i];
            out[i].x = Tr::pack2(opaque(p[i][0].x * a), opaque(p[i][0].y * a));
            out[i].y = Tr::pack2(opaque(p[i][1].x * a), opaque(p[i][1].y * a));
            out[i].z = Tr::pack2(opaque(p[i][2].x * a), opaque(p[i][2].y * a));
            out[i].w = Tr::pack2(opaque(p[i][3].x * a), opaque(p[i][3].y * a));
        }
    }
};

// The first FBA activation fragments (rows xrow0 + 32 f + 0..31) of sub-step j.
template <int FB, int FBA = FB>
__device__ __forceinline__ void read_x(uint4 (&x)[FB], const uint4* sx, int xrow0, int lane, int j) {
    const int ch = 4 * (lane >> 5) + j;
#pragma unroll
    for (int f = 0; f < FBA; ++f) x[f] = sx[swz(xrow0 + f * 32 + (lane & 31), ch)];
}

// MFMAs of one sub-step over the first FBA row fragments; each activation
// fragment is reloaded in place with the fragment of sub-step jn (from buffer
// sx) once its two MFMAs are issued.
template <typename Tr, int FA, int FB, int FBA = FB>
__device__ __forceinline__ void mma_sub(f32x16_t (&acc)[FA][FB], const uint4 (&w)[FA], uint4 (&x)[FB],
                                        const uint4* sx, int xrow0, int lane, int jn) {
    const int ch = 4 * (lane >> 5) + jn;
#pragma unroll
    for (int f = 0; f < FBA; ++f) {
#pragma unroll
        for (int i = 0; i < FA; ++i) acc[i][f] = mfma<Tr>(w[i], x[f], acc[i][f]);
        x[f] = sx[swz(xrow0 + f * 32 + (lane & 31), ch)];
    }
}

// store_tile for the register-weight kernels: 32-bit element offsets from the
// tile's base (the output has fewer than 2^31 elements), one row offset per
// fragment row and compile-time column offsets, so few address registers are
// live. Accumulator row r holds output column r ^ CX (CX = 1: column pairs
// swapped, as the input-gradient kernel's transposed weight reads deliver them).
template <typename Tr, int FA, int FB, int CX = 0>
__device__ __forceinline__ void store_tile_rw(const f32x16_t (&acc)[FA][FB], uint16_t* __restrict__ out, int ld,
                                              int ocol_base, int ocols, int orow_base, int orows,
                                              const uint16_t* __restrict__ bias, int lane) {
    const int c0 = ocol_base + 4 * (lane >> 5);
    float bv[FA][4][4];
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int col = c0 + i * 32 + 8 * q + (e ^ CX);
                bv[i][q][e] = (bias && col < ocols) ? Tr::to_f32(bias[col]) : 0.0f;
            }
    const bool full = ocol_base + FA * 32 <= ocols;
#pragma unroll
    for (int j = 0; j < FB; ++j) {
        const int orow = orow_base + j * 32 + (lane & 31);
        if (orow >= orows) continue;
        uint16_t* dst = out + (orow * ld + c0);
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            f32x16_t a = acc[i][j];
            __asm__ volatile("" : "+v"(a));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = a[4 * q + e] + bv[i][q][e];
                const int dc = i * 32 + 8 * q;
                if (full) {
                    uint2 pk;
                    pk.x = CX ? Tr::pack2(v[1], v[0]) : Tr::pack2(v[0], v[1]);
                    pk.y = CX ? Tr::pack2(v[3], v[2]) : Tr::pack2(v[2], v[3]);
                    *reinterpret_cast<uint2*>(dst + dc) = pk;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (c0 + dc + (e ^ CX) < ocols) dst[dc + (e ^ CX)] = Tr::from_f32(v[e]);
                }
            }
        }
    }
}

// fp32 partial tile of one split for the register-weight kernels: the mapping of
// store_tile_rw (CX as there), 16-byte runs, 32-bit offsets within the split's
// [rows][ld] slice.
template <int FA, int FB, int CX = 0>
__device__ __forceinline__ void store_tile_f32_rw(const f32x16_t (&acc)[FA][FB], float* __restrict__ out, int ld,
                                                  int ocol_base, int ocols, int orow_base, int orows, int lane) {
    const int c0 = ocol_base + 4 * (lane >> 5);
    const bool full = ocol_base + FA * 32 <= ocols;
#pragma unroll
    for (int j = 0; j < FB; ++j) {
        const int orow = orow_base + j * 32 + (lane & 31);
        if (orow >= orows) continue;
        float* dst = out + (orow * ld + c0);
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            f32x16_t a = acc[i][j];
            __asm__ volatile("" : "+v"(a));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int dc = i * 32 + 8 * q;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e ^ CX] = a[4 * q + e];
                if (full) {
                    *reinterpret_cast<float4*>(dst + dc) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (c0 + dc + e < ocols) dst[dc + e] = v[e];
                }
            }
        }
    }
}

// Instruction order of one sub-step of the register-weight kernels: SLOTS
// slots of 1 MFMA, 2 VALU (dequantization) and 1 LDS read (activation
// fragment or level table), an order the compiler's scheduler must follow.
// (MFMA first measured 0-1 % faster in the input gradient than VALU or LDS
// first; the forward is indifferent.)
template <int SLOTS>
__device__ __forceinline__ void rw_slot_pattern() {
#pragma unroll
    for (int k = 0; k < SLOTS; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
}

// Items with at most 64 / 128 valid rows run the 256-row register-weight
// kernels' main loop over 2 / 4 of the 8 row fragments (1: on).
#ifndef STM_SHORT_ITEMS
#define STM_SHORT_ITEMS 1
#endif

template <typename Tr, int BM, int WM>
__global__ __launch_bounds__(256 * WM) void k_gemm_fwd_rw(GemmArgs g) {
    constexpr int BN = 256, NT = 256 * WM, FB = BM / WM / 32;
    const int tid = threadIdx.x, lane0 = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 3, xrow0 = (wave >> 2) * (BM / WM);

    __shared__ float2 lut_all[256 * RW_LUT_COPIES];
    __shared__ uint4 sA0[BM * 8], sA1[BM * 8];

    fill_lut_rw<NT>(lut_all, tid);

    const int64_t K = g.K, N = g.N;
    const int64_t ntm = (g.M + BM - 1) / BM, ntn = (N + BN - 1) / BN, tiles = ntm * ntn;
    int64_t work = tiles * g.num_groups * g.splits, main_work = 0;
    __shared__ GroupedPlan plan;
    bool use_plan = false;
    if constexpr (NT == 256) {
        use_plan = plan_usable(g);
        if (use_plan) {
            build_plan<BM>(g, plan, tid);
            main_work = (int64_t)plan.pre_main[kPlanExperts] * ntn;
            work = main_work + (int64_t)plan.pre_tail[kPlanExperts] * ntn;
        }
    }
    for (int64_t w = blockIdx.x; w < work; w += gridDim.x) {  // work items (tile, expert, split) as in k_gemm_fwd
    int z = 0;
    Group grp;
    int64_t tm, tn;
    if (use_plan) {
        int e;
        plan_item<BM>(plan, g.num_groups, ntn, w, main_work, work, lane0, e, tm, tn);
        grp = plan_group(g, plan, e);
    } else {
        const int64_t wi = item_order(w, work, g.num_groups);
        const int64_t rest = wi / tiles;
        z = (int)(rest / g.num_groups);
        grp = group_of(g, (int)(rest % g.num_groups));
        tile_coords(wi % tiles, ntm, ntn, tm, tn, g.num_groups == 1);
    }
    const int64_t m0 = tm * BM, n0 = tn * BN;
    if (m0 >= grp.rows) continue;

    int s_begin, KT;
    split_range((int)(K / BK), g.splits, z, s_begin, KT);
    const int64_t kbase = (int64_t)s_begin * BK;
    const uint16_t* X = reinterpret_cast<const uint16_t*>(g.a) + grp.row0 * K + kbase;
    const int lane = opaque_lane(lane0);

    RwWeights<Tr> ws;
    ws.bshift = 31 - __builtin_clz(g.blocksize);
    ws.lut_base = (uint32_t)(size_t)((const __attribute__((address_space(3))) float2*)lut_all);
    ws.copy_off = 8u * (uint32_t)(lane & 31);
    const int64_t col_base = n0 + wn * 64;
    ws.packed = grp.packed;
    ws.absmax = grp.absmax;
    ws.kbase = kbase;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int64_t n = col_base + i * 32 + (lane & 31);
        n = n < N ? n : N - 1;
        ws.woff[i] = (uint32_t)(n * (K / 2) + kbase / 2 + 16 * (lane >> 5));
        ws.aoff[i] = (uint32_t)(n * (K >> ws.bshift));
    }
    ActStageS<BM, 4 * WM> as;
    as.init(X, K, m0, grp.rows, sA0, sA1, wave, lane);

    f32x16_t acc[2][FB];
    zero_acc(acc);

    // B[j] = weight fragments of sub-step j. Within step s, slot j is rewritten
    // right after its MFMAs: slot 3 with step s's sub-step 3 (during sub-step
    // 0), slots 0..2 with step s + 1's (during sub-steps 1..3). The table reads
    // of each rewrite are issued one sub-step earlier (into pa / pb, in turn).
    typename RwWeights<Tr>::Raw raw0, raw1;
    uint4 B[4][2];
    uint4 x[FB];
    f32x2_t pa[2][4], pb[2][4];

    // The main loop over the first FBA row fragments of the tile. An item with
    // few valid rows (the last rows of an expert, or of M) runs FBA = 2 or 4
    // (64 or 128 rows): a quarter or half of the MFMAs, the same weight work,
    // and only the waves whose rows hold them copy activations. Rows past the
    // valid ones are never stored.
    // The activation tile of step s + 2 and the packed words of step s + 3 are
    // issued right after the barrier that frees their destination (the buffer
    // step s has just released; the words of step s + 1, whose last table reads
    // go out first), so they have a whole step to land before the next
    // step-end wait (vmcnt(0) counts every load in flight). A step's absmax is
    // loaded, as before, once the absmax it replaces has been used (after
    // sub-step 0). Every load writes the registers the loop carries: no copies.
    auto main_loop = [&](auto fba_tag) {
        constexpr int FBA = decltype(fba_tag)::value;
        // wave w copies the activation rows [w R, w R + R), R = BM / (4 WM)
        const bool copies = FBA == FB || wave * (BM / (4 * WM)) < 32 * FBA;

        // prologue: activation tiles 0 and 1, packed weights of steps 0 and 1;
        // fragments of sub-steps 0..2 of step 0, table reads of its sub-step 3;
        // then step 2's packed words into step 0's registers
        ws.load(0, raw0);
        ws.load(KT > 1 ? BK : 0, raw1);
        if (copies) {
            as.issue(0, 0);
            as.issue(KT > 1 ? BK : 0, 1);
        }
        wait_vmem();
        __syncthreads();  // level table and activation tiles 0 and 1 ready
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            ws.issue(raw0, j, pa);
            RwWeights<Tr>::finish(raw0, pa, B[j]);
        }
        ws.issue(raw0, 3, pa);
        ws.load_words((KT > 2 ? 2 : KT - 1) * (int64_t)BK, raw0);
        read_x<FB, FBA>(x, sA0, xrow0, lane, 0);
        sched_fence();

        auto sub = [&](const uint4 (&w)[2], const uint4* sx, int jn, const typename RwWeights<Tr>::Raw& r_next,
                       int word_next, f32x2_t (&p_next)[2][4], const typename RwWeights<Tr>::Raw& r_cur,
                       const f32x2_t (&p_cur)[2][4], uint4 (&bout)[2]) {
            ws.issue(r_next, word_next, p_next);
            mma_sub<Tr, 2, FB, FBA>(acc, w, x, sx, xrow0, lane, jn);
            RwWeights<Tr>::finish(r_cur, p_cur, bout);
            rw_slot_pattern<2 * FBA>();
            sched_fence();
        };

        // step s: rawc = (packed words of step s + 2, in flight; absmax of step
        // s), rawn = step s + 1; activation tile s in sAc, s + 1 in sAn (in flight)
        auto step = [&](int s, const uint4* sAc, const uint4* sAn, int cbuf, typename RwWeights<Tr>::Raw& rawc,
                        typename RwWeights<Tr>::Raw& rawn) {
            const int s2 = s + 2 < KT ? s + 2 : KT - 1;
            const int s3 = s + 3 < KT ? s + 3 : KT - 1;
            sub(B[0], sAc, 1, rawn, 0, pb, rawc, pa, B[3]);
            ws.load_absmax((int64_t)s2 * BK, rawc);
            sub(B[1], sAc, 2, rawn, 1, pa, rawn, pb, B[0]);
            sub(B[2], sAc, 3, rawn, 2, pb, rawn, pa, B[1]);
            wait_vmem();
            __syncthreads();  // tile s + 1 in sAn; sAc released by every wave
            if (copies) as.issue((int64_t)s2 * BK, cbuf);
            ws.issue(rawn, 3, pa);
            ws.load_words((int64_t)s3 * BK, rawn);
            mma_sub<Tr, 2, FB, FBA>(acc, B[3], x, sAn, xrow0, lane, 0);
            RwWeights<Tr>::finish(rawn, pb, B[2]);
            rw_slot_pattern<2 * FBA>();
            sched_fence();
        };
        int s = 0;
        for (; s + 1 < KT; s += 2) {
            step(s, sA0, sA1, 0, raw0, raw1);
            step(s + 1, sA1, sA0, 1, raw1, raw0);
        }
        if (s < KT) step(s, sA0, sA1, 0, raw0, raw1);
        wait_vmem();  // the loads past the last step (clamped to it) land before the epilogue reuses LDS
    };
    // the item's valid rows decide (uniform over the work-group, so every wave
    // takes the same branch and meets the same barriers)
    const int64_t valid = grp.rows - m0;
    if constexpr (STM_SHORT_ITEMS && FB == 8 && WM == 1) {
        if (valid <= 64)
            main_loop(std::integral_constant<int, 2>{});
        else if (valid <= 128)
            main_loop(std::integral_constant<int, 4>{});
        else
            main_loop(std::integral_constant<int, FB>{});
    } else {
        main_loop(std::integral_constant<int, FB>{});
    }

    const int lane_e = opaque_lane(lane);
    if (g.lora_rank > 0 && z == 0)
        lora_term<Tr, 2, FB>(acc, reinterpret_cast<const uint16_t*>(g.lora_w), col_base, N,
                             reinterpret_cast<const uint16_t*>(g.lora_x) + grp.row0 * g.lora_rank, m0 + xrow0, grp.rows,
                             g.lora_rank, lane_e);
    if (g.splits > 1) {
        store_tile_f32_rw<2, FB>(acc, g.partial + (int64_t)z * g.M * N, (int)N, (int)col_base, (int)N,
                                 (int)(m0 + xrow0), (int)grp.rows, lane_e);
    } else if (STM_RW_LDS_STORE) {
        // the activation buffers stage the output: wave w takes region w of
        // 16 FB rows x 128 bytes (BM / (16 FB) regions per buffer)
        constexpr int RPW = 16 * FB * 8, PER_BUF = BM * 8 / RPW;
        uint4* stage = (wave < PER_BUF ? sA0 + wave * RPW : sA1 + (wave - PER_BUF) * RPW);
        __syncthreads();  // every wave is done reading the activation buffers
        store_tile_lds<Tr, 2, FB>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * N, (int)N, (int)col_base,
                                     (int)N, (int)(m0 + xrow0), (int)grp.rows,
                                     reinterpret_cast<const uint16_t*>(g.bias), lane_e, stage, g.stream_out != 0);
    } else {
        store_tile_rw<Tr, 2, FB>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * N, (int)N, (int)col_base,
                                 (int)N, (int)(m0 + xrow0), (int)grp.rows, reinterpret_cast<const uint16_t*>(g.bias),
                                 lane_e);
    }
    __syncthreads();
    }
}

// ------------------------------ forward, register weights, two waves per SIMD
// The 256 x 256 tile with eight waves: wave w owns the 32 output columns
// [n0 + 32 w, n0 + 32 w + 32) over all 256 rows (8 MFMA tiles, 128
// accumulators), so two waves share each SIMD. The dequantization per MFMA is
// that of k_gemm_fwd_rw (each weight fragment feeds the 8 row tiles), and every
// activation fragment now feeds one MFMA instead of two; in exchange the
// SIMD always has a second wave to issue from while one waits on an LDS read,
// a table lookup or the barrier (with one wave per SIMD those waits stall the
// matrix core). Reduction order, tables and epilogue as in k_gemm_fwd_rw.
#ifndef STM_R8_PATTERN
#define STM_R8_PATTERN 1
#endif
template <int FB>
__device__ __forceinline__ void r8_slot_pattern() {
#if STM_R8_PATTERN
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // the four table reads ride on the first four slots
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
#pragma unroll
    for (int k = 4; k < FB; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#endif
}

template <typename Tr>
__global__ __launch_bounds__(512, 1) void k_gemm_fwd_r8(GemmArgs g) {
    constexpr int BM = 256, BN = 256, NT = 512, FB = BM / 32;
    const int tid = threadIdx.x, lane0 = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    __shared__ float2 lut_all[256 * RW_LUT_COPIES];
    __shared__ uint4 sA0[BM * 8], sA1[BM * 8];

    fill_lut_rw<NT>(lut_all, tid);

    const int64_t K = g.K, N = g.N;
    const int64_t ntm = (g.M + BM - 1) / BM, ntn = (N + BN - 1) / BN, tiles = ntm * ntn;
    const int64_t work = tiles * g.num_groups * g.splits;
    for (int64_t w = blockIdx.x; w < work; w += gridDim.x) {
    const int64_t wi = item_order(w, work, g.num_groups);
    const int64_t rest = wi / tiles;
    const int z = (int)(rest / g.num_groups);
    const Group grp = group_of(g, (int)(rest % g.num_groups));
    int64_t tm, tn;
    tile_coords(wi % tiles, ntm, ntn, tm, tn, g.num_groups == 1);
    const int64_t m0 = tm * BM, n0 = tn * BN;
    if (m0 >= grp.rows) continue;

    int s_begin, KT;
    split_range((int)(K / BK), g.splits, z, s_begin, KT);
    const int64_t kbase = (int64_t)s_begin * BK;
    const uint16_t* X = reinterpret_cast<const uint16_t*>(g.a) + grp.row0 * K + kbase;
    const int lane = opaque_lane(lane0);

    RwWeights<Tr, 1> ws;
    ws.bshift = 31 - __builtin_clz(g.blocksize);
    ws.lut_base = (uint32_t)(size_t)((const __attribute__((address_space(3))) float2*)lut_all);
    ws.copy_off = 8u * (uint32_t)(lane & 31);
    const int64_t col_base = n0 + wave * 32;
    ws.packed = grp.packed;
    ws.absmax = grp.absmax;
    ws.kbase = kbase;
    {
        int64_t n = col_base + (lane & 31);
        n = n < N ? n : N - 1;
        ws.woff[0] = (uint32_t)(n * (K / 2) + kbase / 2 + 16 * (lane >> 5));
        ws.aoff[0] = (uint32_t)(n * (K >> ws.bshift));
    }
    ActStageS<BM, 8> as;
    as.init(X, K, m0, grp.rows, sA0, sA1, wave, lane);

    f32x16_t acc[1][FB];
    zero_acc(acc);

    typename RwWeights<Tr, 1>::Raw raw0, raw1;
    uint4 B[4][1];
    uint4 x[FB];
    f32x2_t pa[1][4], pb[1][4];

    ws.load(0, raw0);
    ws.load(KT > 1 ? BK : 0, raw1);
    as.issue(0, 0);
    wait_vmem();
    __syncthreads();  // level table and activation tile 0 ready
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        ws.issue(raw0, j, pa);
        RwWeights<Tr, 1>::finish(raw0, pa, B[j]);
    }
    ws.issue(raw0, 3, pa);
    read_x<FB>(x, sA0, 0, lane, 0);
    sched_fence();

    auto sub = [&](const uint4 (&wf)[1], const uint4* sx, int jn, const typename RwWeights<Tr, 1>::Raw& r_next,
                   int word_next, f32x2_t (&p_next)[1][4], const typename RwWeights<Tr, 1>::Raw& r_cur,
                   const f32x2_t (&p_cur)[1][4], uint4 (&bout)[1]) {
        ws.issue(r_next, word_next, p_next);
        mma_sub<Tr, 1, FB>(acc, wf, x, sx, 0, lane, jn);
        RwWeights<Tr, 1>::finish(r_cur, p_cur, bout);
        r8_slot_pattern<FB>();
        sched_fence();
    };
    auto step = [&](int s, const uint4* sAc, const uint4* sAn, int nbuf, typename RwWeights<Tr, 1>::Raw& rawc,
                    const typename RwWeights<Tr, 1>::Raw& rawn) {
        const int s1 = s + 1 < KT ? s + 1 : KT - 1;
        const int s2 = s + 2 < KT ? s + 2 : KT - 1;
        as.issue((int64_t)s1 * BK, nbuf);
        sub(B[0], sAc, 1, rawn, 0, pb, rawc, pa, B[3]);
        ws.load((int64_t)s2 * BK, rawc);
        sub(B[1], sAc, 2, rawn, 1, pa, rawn, pb, B[0]);
        sub(B[2], sAc, 3, rawn, 2, pb, rawn, pa, B[1]);
        wait_vmem();
        __syncthreads();  // activation tile s + 1 in sAn; every wave is done reading sAc
        sub(B[3], sAn, 0, rawn, 3, pa, rawn, pb, B[2]);
    };
    int s = 0;
    for (; s + 1 < KT; s += 2) {
        step(s, sA0, sA1, 1, raw0, raw1);
        step(s + 1, sA1, sA0, 0, raw1, raw0);
    }
    if (s < KT) step(s, sA0, sA1, 1, raw0, raw1);

    const int lane_e = opaque_lane(lane);
    if (g.lora_rank > 0 && z == 0)
        lora_term<Tr, 1, FB>(acc, reinterpret_cast<const uint16_t*>(g.lora_w), col_base, N,
                             reinterpret_cast<const uint16_t*>(g.lora_x) + grp.row0 * g.lora_rank, m0, grp.rows,
                             g.lora_rank, lane_e);
    if (g.splits > 1) {
        store_tile_f32_rw<1, FB>(acc, g.partial + (int64_t)z * g.M * N, (int)N, (int)col_base, (int)N, (int)m0,
                                 (int)grp.rows, lane_e);
    } else {
        // the activation buffers stage the output: wave w takes 8 KB (128 rows
        // x 64 bytes per pass), waves 0-3 in sA0, 4-7 in sA1
        constexpr int RPW = 64 * FB;  // uint4 per wave
        uint4* stage = (wave < 4 ? sA0 + wave * RPW : sA1 + (wave - 4) * RPW);
        __syncthreads();  // every wave is done reading the activation buffers
        store_tile_lds<Tr, 1, FB>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * N, (int)N, (int)col_base,
                                     (int)N, (int)m0, (int)grp.rows, reinterpret_cast<const uint16_t*>(g.bias), lane_e,
                                     stage, g.stream_out != 0);
    }
    __syncthreads();
    }
}

// ----------------------------------------------------------------- backward
// dX[m, k] = sum_n dY[m, n] W[n, k]; the tile covers BM rows of dY/dX and BN
// output columns k. Each step reduces over 64 rows n of W; every thread
// dequantizes an 8 (n) x KB (k) block of the W slice and writes it transposed
// (KB columns of 8 consecutive n = one 16-byte chunk each). Piece p of the
// dequantization is the row pair (2p, 2p + 1); the transposed chunks are
// written once all four pairs are done.
template <typename Tr, int KB>
struct BwdStage {
    struct Regs {
        uint32_t q[8];
        float a[8];
    };
    struct Pending {
        float2 c[2][KB / 2];
    };
    const uint8_t* wp;
    const float* wa;
    const float2* lut;
    int64_t row_bytes, kblocks;
    int64_t nbase;  // first reduction index (weight row) of this work-group's step range
    int ng, kg;
    uint32_t col[KB][4];  // col[c][pair] = rows (2 pair, 2 pair + 1) of column c

    __device__ __forceinline__ void load(int s, Regs& w) const {
        const int64_t n0 = nbase + (int64_t)s * BK;  // N % 64 == 0
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const uint8_t* p = wp + (n0 + r) * row_bytes;
            if constexpr (KB == 8)
                w.q[r] = *reinterpret_cast<const uint32_t*>(p);
            else
                w.q[r] = *reinterpret_cast<const uint16_t*>(p);
            w.a[r] = wa[(n0 + r) * kblocks];
        }
    }
    __device__ __forceinline__ void issue(const Regs& w, int pair, Pending& p) const {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int b = 0; b < KB / 2; ++b) p.c[h][b] = lut[((w.q[2 * pair + h] >> (8 * b)) & 0xFFu) * LUT_COPIES];
    }
    __device__ __forceinline__ void finish(const Regs& w, int pair, const Pending& p, uint4*) {
        float v[2][KB];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float a = w.a[2 * pair + h];
#pragma unroll
            for (int b = 0; b < KB / 2; ++b) {
                v[h][2 * b] = opaque(p.c[h][b].x * a);
                v[h][2 * b + 1] = opaque(p.c[h][b].y * a);
            }
        }
#pragma unroll
        for (int c = 0; c < KB; ++c) col[c][pair] = Tr::pack2(v[0][c], v[1][c]);
    }
    __device__ __forceinline__ void flush(uint4* dst) const {
#pragma unroll
        for (int c = 0; c < KB; ++c) dst[swz(kg * KB + c, ng)] = make_uint4(col[c][0], col[c][1], col[c][2], col[c][3]);
    }
    __device__ __forceinline__ void store_all(const Regs& w, uint4* dst) {
#pragma unroll
        for (int pair = 0; pair < 4; ++pair) {
            Pending p;
            issue(w, pair, p);
            finish(w, pair, p, dst);
        }
        flush(dst);
    }
};

template <typename Tr, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM* WN * 64) void k_gemm_bwd(GemmArgs g) {
    constexpr int NW = WM * WN, NT = NW * 64;
    constexpr int FX = BM / WM / 32;
    constexpr int FW = BN / WN / 32;
    constexpr int KB = 8 * BN / NT;  // k columns per thread block: 8 n-groups x (BN / KB) k-groups = NT
    static_assert(BM % (8 * NW) == 0 && (KB == 4 || KB == 8), "tile / wave mismatch");
    __shared__ float2 lut_all[256 * LUT_COPIES];
    __shared__ uint4 sA0[BM * 8], sA1[BM * 8];
    __shared__ uint4 sB0[BN * 8], sB1[BN * 8];

    // (large tiles) the wave index as a uniform value: wave-derived offsets then
    // live in SGPRs instead of taking VGPRs from the accumulators' neighbours
    constexpr bool kLargeAcc = (BM / WM / 32) * (BN / WN / 32) >= 8;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = kLargeAcc ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    fill_lut<NT>(lut_all, tid);

    const int64_t K = g.K, N = g.N;
    const int64_t ntm = (g.M + BM - 1) / BM, ntk = (K + BN - 1) / BN, tiles = ntm * ntk;
    const int64_t work = tiles * g.num_groups * g.splits;
    for (int64_t w = blockIdx.x; w < work; w += gridDim.x) {  // work items as in k_gemm_fwd
    const int64_t wi = item_order(w, work, g.num_groups);
    const int64_t rest = wi / tiles;
    const int z = (int)(rest / g.num_groups);
    const Group grp = group_of(g, (int)(rest % g.num_groups));
    int64_t tm, tk;
    tile_coords(wi % tiles, ntm, ntk, tm, tk, g.num_groups == 1);
    const int64_t m0 = tm * BM, k0 = tk * BN;
    if (m0 >= grp.rows) continue;

    int s_begin, NT_steps;
    split_range((int)(N / BK), g.splits, z, s_begin, NT_steps);
    const uint16_t* __restrict__ DY = reinterpret_cast<const uint16_t*>(g.a) + grp.row0 * N + (int64_t)s_begin * BK;
    const int64_t kblocks = K / g.blocksize;
    const int bshift = ilog2(g.blocksize);

    BwdStage<Tr, KB> ws;
    ws.nbase = (int64_t)s_begin * BK;
    ws.ng = tid & 7;
    ws.kg = tid >> 3;
    int64_t kc = k0 + ws.kg * KB;
    kc = kc < K ? kc : K - KB;  // columns past K only feed outputs that are never stored
    ws.wp = grp.packed + (int64_t)(ws.ng * 8) * (K / 2) + kc / 2;
    ws.wa = grp.absmax + (int64_t)(ws.ng * 8) * kblocks + (kc >> bshift);
    ws.lut = lut_all + (lane & (LUT_COPIES - 1));
    ws.row_bytes = K / 2;
    ws.kblocks = kblocks;

    f32x16_t acc[FW][FX];
    zero_acc(acc);
    run_pipeline<Tr, BM, BN, WM, WN, FW, FX>(acc, DY, N, m0, grp.rows, NT_steps, sA0, sA1, sB0, sB1, ws, wave, lane);

    const int64_t col_base = k0 + wn * (BN / WN), row_base = m0 + wm * (BM / WM);
    const int lane_e = FW * FX >= 8 ? opaque_lane(lane) : lane;
    if (g.lora_rank > 0 && z == 0)
        lora_term<Tr, FW, FX>(acc, reinterpret_cast<const uint16_t*>(g.lora_w), col_base, K,
                              reinterpret_cast<const uint16_t*>(g.lora_x) + grp.row0 * g.lora_rank, row_base,
                              grp.rows, g.lora_rank, lane_e);
    if (g.splits > 1)
        store_tile_f32<FW, FX>(acc, g.partial + (int64_t)z * g.M * K, K, col_base, K, row_base, grp.rows, lane_e);
    else
        store_tile<Tr, FW, FX>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * K, K, col_base, K, row_base,
                               grp.rows, nullptr, lane_e);
    __syncthreads();
    }
}

// -------------------------------------------- input gradient, register weights
// dX tile BM x 256 (rows m x output columns k) with four waves; wave w owns the
// 64 output columns [k0 + 64 w, k0 + 64 w + 64) over all BM rows, so, as in
// k_gemm_fwd_rw, each wave dequantizes its own weight fragments into MFMA
// operand registers. The MFMA's weight-side operand needs 8 consecutive
// reduction indices n of one column k per lane -- a column of the row-major
// packed weight. The packed tile (64 rows x 256 columns = 8 KB per step) is
// copied into LDS and read back with ds_read_b64_tr_b4: within a 16-lane group,
// lane i points at 16 packed columns of row i, and lane c receives nibble c of
// the 16 rows, row r in nibble r -- 16 consecutive n of one column. Nibble c is
// the low nibble of byte c / 2 for even c, and packed NF4 keeps the even column
// in the high nibble, so lane c holds column c ^ 1: the accumulators' rows are
// output columns in swapped pairs, undone by the store (and the LoRA term reads
// its weight-side rows in the same order).
//
// Reduction order in a 64-deep step: lane half h at MFMA sub-step j takes rows
// N(j, h) = 16 (2 (j / 2) + h) + 8 (j % 2) + (0..7); the activation (dY)
// operand of lane (m, h) is LDS chunk N(j, h) / 8 of row m. Transposed read T
// of fragment i (lanes of half h: rows 16 (2 T + h) + 0..15) covers sub-steps
// 2 T (nibbles 0..7) and 2 T + 1 (nibbles 8..15). The absmax of a weight row
// differs per n, so the step's absmax values [4 column blocks][64 rows] are
// staged in LDS (1 KB) and each sub-step reads its 8 per half as two broadcast
// 16-byte reads.
//
// Step s: copy dY(s + 1) and the packed tile of step s + 2 into LDS and load the
// absmax of step s + 2; sub-steps 0..2 compute while step s + 1's fragments are
// dequantized (transposed reads of its tile were done one step earlier); wait
// for the copies, store the absmax, barrier; sub-step 3, during which step
// s + 2's tile (published by that barrier) is read transposed. Runs the 256 x 256
// input gradients, unsplit or split into ranges of >= 32 steps (a split's
// work-group stores its fp32 partial tile).
template <typename Tr>
struct RwWeightsT {
    struct Raw {
        uint2 t[2][2];  // [fragment][transposed read T]
    };
    uint32_t lut_base, copy_off;

    // transposed reads of one packed tile (buffer at LDS byte address tile)
    __device__ __forceinline__ static void read(uint32_t tile, const uint32_t (&addr)[2][2], Raw& r) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int T = 0; T < 2; ++T) {
                const v2i32_t v = __builtin_amdgcn_ds_read_tr4_b64_v2i32(
                    (__attribute__((address_space(3))) v2i32_t*)(size_t)(tile + addr[i][T]));
                r.t[i][T] = make_uint2((uint32_t)v.x, (uint32_t)v.y);
            }
    }
    // table reads of sub-step j (both fragments) and the sub-step's 8 absmax values
    __device__ __forceinline__ void issue(const Raw& r, int j, f32x2_t (&p)[2][4], uint32_t absrow,
                                          f32x4_t (&a)[2]) const {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t x = (j & 1) ? r.t[i][j >> 1].y : r.t[i][j >> 1].x;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t addr = __builtin_amdgcn_perm(copy_off, x, 0x0C0C0004u | ((uint32_t)b << 8));
                p[i][b] = *(const __attribute__((address_space(3))) f32x2_t*)(size_t)(lut_base + addr);
            }
        }
        a[0] = *(const __attribute__((address_space(3))) f32x4_t*)(size_t)absrow;
        a[1] = *(const __attribute__((address_space(3))) f32x4_t*)(size_t)(absrow + 16);
    }
    // byte b of a transposed word holds rows 2 b (low nibble) and 2 b + 1
    __device__ __forceinline__ static void finish(const f32x2_t (&p)[2][4], const f32x4_t (&a)[2],
                                                  uint4 (&out)[2]) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            out[i].x = Tr::pack2(opaque(p[i][0].y * a[0].x), opaque(p[i][0].x * a[0].y));
            out[i].y = Tr::pack2(opaque(p[i][1].y * a[0].z), opaque(p[i][1].x * a[0].w));
            out[i].z = Tr::pack2(opaque(p[i][2].y * a[1].x), opaque(p[i][2].x * a[1].y));
            out[i].w = Tr::pack2(opaque(p[i][3].y * a[1].z), opaque(p[i][3].x * a[1].w));
        }
    }
};

template <typename Tr, int BM>
__global__ __launch_bounds__(256) void k_gemm_bwd_rw(GemmArgs g) {
    constexpr int BN = 256, NT = 256, FB = BM / 32;
    const int tid = threadIdx.x, lane0 = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    __shared__ float2 lut_all[256 * RW_LUT_COPIES];
    __shared__ uint4 sA0[BM * 8], sA1[BM * 8];  // dY tiles [m][64 n]
    __shared__ uint4 sW0[64 * 8], sW1[64 * 8];  // packed weight tiles [64 n][256 k / 2]
    __shared__ float sS[3][4 * 64];             // absmax [column block][64 n], step s in sS[s % 3]

    fill_lut_rw<NT>(lut_all, tid);

    const int64_t K = g.K, N = g.N;
    const int64_t ntm = (g.M + BM - 1) / BM, ntk = (K + BN - 1) / BN, tiles = ntm * ntk;
    int64_t work = tiles * g.num_groups * g.splits, main_work = 0;
    __shared__ GroupedPlan plan;
    const bool use_plan = plan_usable(g);
    if (use_plan) {
        build_plan<BM>(g, plan, tid);
        main_work = (int64_t)plan.pre_main[kPlanExperts] * ntk;
        work = main_work + (int64_t)plan.pre_tail[kPlanExperts] * ntk;
    }
    for (int64_t w = blockIdx.x; w < work; w += gridDim.x) {  // items (tile, expert, split)
    int z = 0;
    Group grp;
    int64_t tm, tk;
    if (use_plan) {
        int e;
        plan_item<BM>(plan, g.num_groups, ntk, w, main_work, work, lane0, e, tm, tk);
        grp = plan_group(g, plan, e);
    } else {
        const int64_t wi = item_order(w, work, g.num_groups);
        const int64_t rest = wi / tiles;
        z = (int)(rest / g.num_groups);
        grp = group_of(g, (int)(rest % g.num_groups));
        tile_coords(wi % tiles, ntm, ntk, tm, tk, g.num_groups == 1);
    }
    const int64_t m0 = tm * BM, k0 = tk * BN;
    if (m0 >= grp.rows) continue;

    int s_begin, KT;
    split_range((int)(N / BK), g.splits, z, s_begin, KT);
    const int lane = opaque_lane(lane0);
    const int bshift = 31 - __builtin_clz(g.blocksize);
    const int64_t col_base = k0 + wave * 64;

    // dY tile copies (as the forward's activation copies, leading dimension N)
    ActStageS<BM, 4> as;
    as.init(reinterpret_cast<const uint16_t*>(g.a) + grp.row0 * N + (int64_t)s_begin * BK, N, m0, grp.rows, sA0, sA1,
            wave, lane);

    // packed-tile copies: slot S = 64 (4 i + wave) + lane of 512 16-byte slots,
    // row r = S / 8, LDS chunk S % 8 holds packed chunk (S % 8) ^ key(r) of row r
    // (columns past K re-read the row's last chunk; they feed unstored outputs)
    uint32_t woff[2], wlds[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int S0 = 64 * (4 * i + wave);
        const int r = (S0 + lane) >> 3, cs = lane & 7;
        int64_t cb = k0 / 2 + 16 * (cs ^ swz_key(r));
        cb = cb + 16 <= K / 2 ? cb : K / 2 - 16;
        woff[i] = (uint32_t)(r * (K / 2) + cb);
        wlds[i] = (uint32_t)__builtin_amdgcn_readfirstlane(lds_offset(sW0 + S0));
    }
    const uint32_t wstride = (uint32_t)(lds_offset(sW1) - lds_offset(sW0));
    // absmax staging: lane = row n, wave = 64-column block of the tile
    int64_t kcol = k0 + 64 * wave;
    kcol = kcol < K ? kcol : K - 64;
    const uint32_t aoff = (uint32_t)(lane * (K >> bshift) + (kcol >> bshift));
    const uint32_t sS0 = (uint32_t)(size_t)((__attribute__((address_space(3))) float*)&sS[0][0]);

    // transposed-read addresses of fragment i, read T (relative to a tile buffer)
    const int h = lane >> 5, cbk = (lane >> 4) & 1, rr = lane & 15;
    uint32_t traddr[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const int r = 16 * (2 * T + h) + rr;
            const int c = 2 * wave + i;
            traddr[i][T] = (uint32_t)(16 * (r * 8 + (c ^ swz_key(r))) + 8 * cbk);
        }
    const uint32_t tile0 = lds_offset(sW0), tile1 = lds_offset(sW1);

    RwWeightsT<Tr> ws;
    ws.lut_base = (uint32_t)(size_t)((const __attribute__((address_space(3))) float2*)lut_all);
    ws.copy_off = 8u * (uint32_t)(lane & 31);
    // absmax row address of sub-step j, half h, in buffer b
    auto absrow = [&](int b, int j) {
        return sS0 + 4u * (uint32_t)(256 * b + 64 * wave + 16 * (2 * (j >> 1) + h) + 8 * (j & 1));
    };

    const uint8_t* pk = grp.packed + (int64_t)s_begin * BK * (K / 2);  // the split's first weight row
    const float* am = grp.absmax + (int64_t)s_begin * BK * (K >> bshift);
    auto copy_w = [&](int s, int buf) {  // packed tile of step s -> sW[buf]
        const uint8_t* base = pk + (int64_t)s * BK * (K / 2);
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16_s(base, woff[i], wlds[i] + (uint32_t)buf * wstride);
    };
    auto load_abs = [&](int s) { return am[(int64_t)s * BK * (K >> bshift) + aoff]; };
    auto store_abs = [&](int buf, float v) {
        *(__attribute__((address_space(3))) float*)(size_t)(sS0 + 4u * (uint32_t)(256 * buf + 64 * wave + lane)) = v;
    };

    f32x16_t acc[2][FB];
    zero_acc(acc);
    typename RwWeightsT<Tr>::Raw raw0, raw1;
    uint4 B[4][2];
    uint4 x[FB];
    f32x2_t pa[2][4], pb[2][4];
    f32x4_t aa[2], ab[2];
    const int xh = lane >> 5;
    auto xch = [&](int j) { return 4 * (j >> 1) + 2 * xh + (j & 1); };

    // The main loop over the first FBA row fragments (as in k_gemm_fwd_rw: an
    // item with at most 64 / 128 valid rows runs 2 / 4 of them, and only the
    // waves whose rows hold them copy dY). Each step's loads are issued right
    // after the barrier that frees their destination, so each has a whole step
    // to land before the next step-end wait: dY of step s + 2 into the dY buffer
    // step s has released, the packed tile of step s + 3 into the tile buffer
    // whose tile (s + 1) was read into registers a barrier ago, and the absmax
    // of step s + 3 into a register, stored to its LDS buffer before the next
    // barrier.
    auto main_loop = [&](auto fba_tag) {
        constexpr int FBA = decltype(fba_tag)::value;
        // wave w copies the dY rows [w BM / 4, (w + 1) BM / 4)
        const bool copies = FBA == FB || wave * (BM / 4) < 32 * FBA;

        // prologue: dY(0) and dY(1), packed tiles of steps 0 and 1, absmax of
        // steps 0 and 1; fragments of sub-steps 0..2 of step 0, table reads of its
        // sub-step 3; then the tile and absmax of step 2
        {
            const float a0 = load_abs(0), a1 = load_abs(KT > 1 ? 1 : 0);
            if (copies) {
                as.issue(0, 0);
                as.issue(KT > 1 ? BK : 0, 1);
            }
            copy_w(0, 0);
            copy_w(KT > 1 ? 1 : 0, 1);
            wait_vmem();
            store_abs(0, a0);
            store_abs(1, a1);  // absmax of step s in buffer s % 3
        }
        __syncthreads();  // level table, dY(0), dY(1), tiles 0 and 1, absmax 0 and 1 ready
        RwWeightsT<Tr>::read(tile0, traddr, raw0);
        RwWeightsT<Tr>::read(tile1, traddr, raw1);
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            ws.issue(raw0, j, pa, absrow(0, j), aa);
            RwWeightsT<Tr>::finish(pa, aa, B[j]);
        }
        ws.issue(raw0, 3, pa, absrow(0, 3), aa);
        // activation fragments of sub-step 0
#pragma unroll
        for (int f = 0; f < FBA; ++f) x[f] = sA0[swz(f * 32 + (lane & 31), xch(0))];
        __syncthreads();  // every wave has read tile 0 before its buffer takes tile 2
        copy_w(KT > 2 ? 2 : KT - 1, 0);
        float a_next = load_abs(KT > 2 ? 2 : KT - 1);

        auto sub = [&](const uint4 (&wf)[2], const uint4* sx, int jn, const typename RwWeightsT<Tr>::Raw& r_next,
                       int j_next, uint32_t arow_next, f32x2_t (&p_next)[2][4], f32x4_t (&a_next)[2],
                       const f32x2_t (&p_cur)[2][4], const f32x4_t (&a_cur)[2], uint4 (&bout)[2]) {
            ws.issue(r_next, j_next, p_next, arow_next, a_next);
            const int ch = xch(jn);
#pragma unroll
            for (int f = 0; f < FBA; ++f) {
                acc[0][f] = mfma<Tr>(wf[0], x[f], acc[0][f]);
                acc[1][f] = mfma<Tr>(wf[1], x[f], acc[1][f]);
                x[f] = sx[swz(f * 32 + (lane & 31), ch)];
            }
            RwWeightsT<Tr>::finish(p_cur, a_cur, bout);
            rw_slot_pattern<2 * FBA>();
            sched_fence();
        };

        // step s: rawc = transposed tile of step s (its sub-step 3 not yet made),
        // rawn = step s + 1; dY(s) in sAc, dY(s + 1) in sAn (in flight); tile s + 2
        // in flight into buffer cur; a_next = absmax of step s + 2 (in flight);
        // absmax buffers rotate over three (step s + 1 in a1, step s + 2 into
        // a2buf, whose last reader, step s - 2's sub-step 3, is a barrier behind)
        auto step = [&](int s, const uint4* sAc, const uint4* sAn, int cur, typename RwWeightsT<Tr>::Raw& rawc,
                        const typename RwWeightsT<Tr>::Raw& rawn) {
            const int s2 = s + 2 < KT ? s + 2 : KT - 1;
            const int s3 = s + 3 < KT ? s + 3 : KT - 1;
            const int a1 = (s + 1) % 3, a2buf = (s + 2) % 3;
            sub(B[0], sAc, 1, rawn, 0, absrow(a1, 0), pb, ab, pa, aa, B[3]);
            sub(B[1], sAc, 2, rawn, 1, absrow(a1, 1), pa, aa, pb, ab, B[0]);
            sub(B[2], sAc, 3, rawn, 2, absrow(a1, 2), pb, ab, pa, aa, B[1]);
            wait_vmem();
            store_abs(a2buf, a_next);
            __syncthreads();  // dY(s + 1), tile and absmax of step s + 2 ready; sAc free
            RwWeightsT<Tr>::read(cur ? tile1 : tile0, traddr, rawc);  // step s + 2's tile into the freed registers
            if (copies) as.issue((int64_t)s2 * BK, cur);
            copy_w(s3, cur ^ 1);  // tile s + 1 left that buffer a barrier ago
            a_next = load_abs(s3);
            sub(B[3], sAn, 0, rawn, 3, absrow(a1, 3), pa, aa, pb, ab, B[2]);
        };
        int s = 0;
        for (; s + 1 < KT; s += 2) {
            step(s, sA0, sA1, 0, raw0, raw1);
            step(s + 1, sA1, sA0, 1, raw1, raw0);
        }
        if (s < KT) step(s, sA0, sA1, 0, raw0, raw1);
        wait_vmem();  // the loads past the last step (clamped to it) land before the epilogue reuses LDS
    };
    const int64_t valid = grp.rows - m0;  // uniform over the work-group
    if constexpr (STM_SHORT_ITEMS && FB == 8) {
        if (valid <= 64)
            main_loop(std::integral_constant<int, 2>{});
        else if (valid <= 128)
            main_loop(std::integral_constant<int, 4>{});
        else
            main_loop(std::integral_constant<int, FB>{});
    } else {
        main_loop(std::integral_constant<int, FB>{});
    }

    const int lane_e = opaque_lane(lane);
    if (g.lora_rank > 0 && z == 0)
        lora_term<Tr, 2, FB, 1>(acc, reinterpret_cast<const uint16_t*>(g.lora_w), col_base, K,
                                reinterpret_cast<const uint16_t*>(g.lora_x) + grp.row0 * g.lora_rank, m0, grp.rows,
                                g.lora_rank, lane_e);
    if (g.splits > 1) {
        store_tile_f32_rw<2, FB, 1>(acc, g.partial + (int64_t)z * g.M * K, (int)K, (int)col_base, (int)K, (int)m0,
                                    (int)grp.rows, lane_e);
    } else if (STM_RW_LDS_STORE) {
        // the dY buffers stage the output as in k_gemm_fwd_rw (every copy of the
        // last step was awaited before its barrier)
        constexpr int RPW = 16 * FB * 8, PER_BUF = BM * 8 / RPW;
        uint4* stage = (wave < PER_BUF ? sA0 + wave * RPW : sA1 + (wave - PER_BUF) * RPW);
        __syncthreads();  // every wave is done reading the dY buffers
        store_tile_lds<Tr, 2, FB, 1>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * K, (int)K, (int)col_base,
                                        (int)K, (int)m0, (int)grp.rows, nullptr, lane_e, stage, g.stream_out != 0);
    } else {
        store_tile_rw<Tr, 2, FB, 1>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * K, (int)K, (int)col_base,
                                    (int)K, (int)m0, (int)grp.rows, nullptr, lane_e);
    }
    __syncthreads();
    }
}

// ------------------------------------------------------------ small-M forward
// Y[M, N] = X[M, K] . W[N, K]^T for M <= 64 rows (decode-sized batches),
// bound by dequantizing the streamed weight. A work-group owns 32 weight rows
// per wave (two v_mfma_f32_16x16x32 tiles of weight rows x activation rows,
// 16 MB activation rows; GvCfg) over one reduction range, walked in groups of
// GK = 256 or 128 (always 128 above 32 rows, whose larger activation buffers
// must fit; at 17-32 rows the host picks the layout).
// Every operand reaches LDS through lane-contiguous global -> LDS copies
// (whole 64- or 128-byte row pieces), double-buffered, one barrier per group:
//  - packed weight: each wave copies its own 32 rows x GK / 2 bytes (PW
//    16-byte pieces per row); piece p of row r sits in slot
//    p ^ ((r >> WSH) % PW), so the MFMA-layout reads (16 lanes = 16 rows,
//    same piece) hit all banks once;
//  - absmax: each wave copies its rows' blocks of the group (dword copies);
//  - activations: the group's <= 16 MB rows x 2 GK bytes, shared by the
//    waves, piece p of row m in slot p ^ (m % 16).
// Within a group, 128-deep chunk c: lane (r = lane % 16, h = lane / 16)
// reads 16 packed bytes (k = 128 c + 32 h + 0..31) of row r of each tile and
// their absmax, dequantizes in registers with the level table as in
// k_gemm_fwd_rw, and MFMA q (0..3) takes k = 128 c + 32 h + 8 q + (0..7) from
// both operands. Past K (K % GK != 0) the copies read valid addresses and
// the lanes use a zero scale and zero activations. Reduction ranges (splits)
// write fp32 partials [split][m][n] that k_split_reduce sums (with bias and
// the LoRA term); with one range the output (plus bias) is stored directly.
// Work-group shape: WAVES waves of 32 weight rows (two 16-row MFMA tiles)
// each. MB = 1: 8 waves (256 rows); MB = 2: 6 waves (192 rows), so the
// doubled activation buffers still fit beside the 64 KB level table (150 KB
// of LDS), or 8 waves over groups of 128 (116 KB); MB = 3 and 4 (33-48 and
// 49-64 rows): 8 waves over groups of 128 (124 and 132 KB).
template <int MB, int GK_>
struct GvCfg {
    static constexpr int GK = GK_;                       // reduction depth of a group
    static constexpr int WAVES = MB == 2 && GK == 256 ? 6 : 8, R = 2, RW = 32, ROWS = RW * WAVES, XR = 16 * MB;
    static constexpr int PW = GK / 32, PX = GK / 8;      // 16-byte pieces of a weight row, an activation row
    static constexpr int NCH = GK / 128, NFL = GK / 64;  // 128-deep chunks; absmax per row (blocksize >= 64)
    static constexpr int WSH = PW == 8 ? 1 : 2;          // weight slot swizzle: piece ^ ((row >> WSH) % PW)
    static constexpr int kLut = 256 * RW_LUT_COPIES * 8, kX = XR * PX * 16, kW = ROWS * PW * 16, kA = ROWS * NFL * 4;
    static constexpr int kLds = kLut + 2 * (kX + kW + kA);
    static_assert(kLds <= 160 * 1024, "LDS");
    static_assert((PW << WSH) == 16 && RW * PW % 64 == 0 && XR * PX % 64 == 0, "copy shapes");
};
constexpr int GV_GK = 256;  // group depth of k_gemv_ks

template <typename Tr, int MB, int GK, bool GROUPED = false>
__global__ __launch_bounds__((64 * GvCfg<MB, GK>::WAVES)) void k_gemv_fwd(GemmArgs g, int groups_per_split) {
    using C = GvCfg<MB, GK>;
    constexpr int R = C::R, WAVES = C::WAVES;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // one LDS array, the level table first (at address 0, so a perm-built
    // table address needs no base added)
    __shared__ __align__(16) uint8_t smem[C::kLds];
    float2* lut_all = reinterpret_cast<float2*>(smem);
    auto sx = [&](int buf) { return reinterpret_cast<uint4*>(smem + C::kLut + buf * C::kX); };
    auto sw = [&](int buf) {
        return reinterpret_cast<uint4*>(smem + C::kLut + 2 * C::kX + buf * C::kW) + wave * (C::RW * C::PW);
    };
    auto sa = [&](int buf) {
        return reinterpret_cast<float*>(smem + C::kLut + 2 * (C::kX + C::kW) + buf * C::kA) + wave * (C::RW * C::NFL);
    };

    const int64_t K = g.K, N = g.N;
    const int bshift = 31 - __builtin_clz(g.blocksize);
    const int nfl = (C::GK >> bshift) > 0 ? (C::GK >> bshift) : 1;  // absmax per row per group
    const int64_t kblocks = K >> bshift;
    const int ngroups = (int)((K + C::GK - 1) / C::GK);
    // GROUPED: expert blockIdx.y (one reduction range): its rows from the
    // offsets, at most g.M (the caller's bound, at most 16 MB rows), its
    // weight and its output rows; a work-group of an empty expert leaves
    // before any barrier
    int64_t M = g.M;
    const uint16_t* xa = reinterpret_cast<const uint16_t*>(g.a);
    const uint8_t* wpk = g.packed;
    const float* wab = g.absmax;
    uint16_t* yo = reinterpret_cast<uint16_t*>(g.out);
    int z = blockIdx.y;
    if constexpr (GROUPED) {
        const Group gr = group_of(g, (int)blockIdx.y);
        M = gr.rows < 0 ? 0 : gr.rows < g.M ? gr.rows : g.M;
        if (M <= 0) return;
        xa += gr.row0 * K;
        yo += gr.row0 * N;
        wpk = gr.packed;
        wab = gr.absmax;
        z = 0;
    }
    const int g_begin = z * groups_per_split;
    const int g_end = g_begin + groups_per_split < ngroups ? g_begin + groups_per_split : ngroups;
    const int64_t nw0 = (int64_t)blockIdx.x * C::ROWS + wave * C::RW;  // this wave's first weight row

    // copy sources (per lane; group offsets added per copy): weight copy i
    // covers rows 64 / PW i + lane / PW, slot lane % PW of each
    constexpr int PW = C::PW, WC = C::RW * PW / 64;
    auto wslot_piece = [](int row, int slot) { return slot ^ ((row >> C::WSH) & (PW - 1)); };
    const uint8_t* wsrc[WC];
#pragma unroll
    for (int i = 0; i < WC; ++i) {
        const int row = 64 / PW * i + lane / PW;
        const int64_t n = nw0 + row < N ? nw0 + row : N - 1;
        wsrc[i] = wpk + n * (K / 2) + 16 * wslot_piece(row, lane % PW);
    }
    const int a_rows_per_copy = 64 / nfl, a_copies = (C::RW * nfl + 63) / 64;  // <= R
    const float* asrc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int64_t n0 = nw0 + lane / nfl + i * a_rows_per_copy;
        asrc[i] = wab + (n0 < N ? n0 : N - 1) * kblocks;
    }
    const int aj = lane % nfl;
    // activations: XR PX / 64 copies of 64 / PX rows each, copy ix by wave ix % WAVES
    constexpr int PX = C::PX, XI = C::XR * PX / 64, XC = (XI + WAVES - 1) / WAVES;
    const uint16_t* xsrc[XC];
    int xpiece[XC];
#pragma unroll
    for (int j = 0; j < XC; ++j) {
        const int xm = 64 / PX * (wave + j * WAVES) + lane / PX;  // activation row this lane copies
        xsrc[j] = xa + (xm < M ? xm : M - 1) * K;
        xpiece[j] = (lane % PX) ^ (xm & 15);
    }

    auto uniform = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane(v); };
    auto copy_group = [&](int grp, int buf) {
        const int64_t kg = (int64_t)grp * C::GK;
#pragma unroll
        for (int i = 0; i < WC; ++i) {
            // bytes past the row (K % GK != 0) read the row start instead
            const int piece = wslot_piece(64 / PW * i + lane / PW, lane % PW);
            const uint8_t* src = kg / 2 + 16 * piece < K / 2 ? wsrc[i] + kg / 2 : wsrc[i] - 16 * piece;
            dma16(src, uniform(lds_offset(sw(buf) + i * 64)));
        }
        const int64_t b0 = kg >> bshift;
        const int64_t blk = b0 + aj < kblocks ? b0 + aj : kblocks - 1;
#pragma unroll
        for (int i = 0; i < R; ++i)
            if (i < a_copies)
                dma4(asrc[i] + blk,
                     uniform((uint32_t)(size_t)((const __attribute__((address_space(3))) float*)(sa(buf) + i * 64))));
#pragma unroll
        for (int j = 0; j < XC; ++j)
            if (wave + j * WAVES < XI) {
                const int64_t k = kg + 8 * xpiece[j];
                dma16(xsrc[j] + (k < K ? k : 0), uniform(lds_offset(sx(buf) + (wave + j * WAVES) * 64)));
            }
    };

    const int r = lane & 15, h = lane >> 4;
    const uint32_t copy_off = 8u * (uint32_t)(lane & 31);
    f32x4_t acc[R][MB];
#pragma unroll
    for (int t = 0; t < R; ++t)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[t][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // one group: work items (chunk c, tile t) in order i = R c + t; the table
    // reads of item i + 1 are written before item i's products, conversions and
    // MFMAs, with no scheduling fence between items (the compiler's
    // interleaving across items measured 2-10 % faster than fenced items).
    // TAIL (the group that reaches past K) zeroes the activations and the
    // scale of lanes whose k is past K.
    auto compute = [&](int buf, int grp, auto tail_c) {
        constexpr bool TAIL = decltype(tail_c)::value;
        uint4 xv[C::NCH][MB][4], qv[C::NCH * R];
        float av[C::NCH * R];
#pragma unroll
        for (int c = 0; c < C::NCH; ++c) {
            const bool ok = !TAIL || (int64_t)grp * C::GK + 128 * c + 32 * h < K;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int xr = 16 * mb + r;
                    const uint4 v = sx(buf)[xr * PX + ((16 * c + 4 * h + q) ^ r)];
                    xv[c][mb][q] = ok ? v : make_uint4(0, 0, 0, 0);
                }
            const int blk = (128 * c + 32 * h) >> bshift;
#pragma unroll
            for (int t = 0; t < R; ++t) {
                const int row = 16 * t + r;
                qv[R * c + t] = sw(buf)[row * PW + wslot_piece(row, 4 * c + h)];
                const float a = sa(buf)[row * nfl + blk];
                av[R * c + t] = ok ? a : 0.0f;
            }
        }
        f32x2_t p[2][4][4];
        auto issue = [&](int i, f32x2_t (&pp)[4][4]) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t word = q == 0 ? qv[i].x : q == 1 ? qv[i].y : q == 2 ? qv[i].z : qv[i].w;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t addr = __builtin_amdgcn_perm(copy_off, word, 0x0C0C0004u | ((uint32_t)b << 8));
                    pp[q][b] = *(const __attribute__((address_space(3))) f32x2_t*)(size_t)addr;
                }
            }
        };
        issue(0, p[0]);
#pragma unroll
        for (int i = 0; i < C::NCH * R; ++i) {
            if (i + 1 < C::NCH * R) issue(i + 1, p[(i + 1) & 1]);
            const int c = i / R, t = i % R;
            const float a = av[i];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x2_t(&pq)[4] = p[i & 1][q];
                uint4 w;
                w.x = Tr::pack2(opaque(pq[0].x * a), opaque(pq[0].y * a));
                w.y = Tr::pack2(opaque(pq[1].x * a), opaque(pq[1].y * a));
                w.z = Tr::pack2(opaque(pq[2].x * a), opaque(pq[2].y * a));
                w.w = Tr::pack2(opaque(pq[3].x * a), opaque(pq[3].y * a));
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) acc[t][mb] = mfma16<Tr>(w, xv[c][mb][q], acc[t][mb]);
            }
        }
    };

    if (g_begin < g_end) copy_group(g_begin, 0);  // in flight while the level table is filled
    fill_lut_rw<64 * WAVES>(lut_all, tid);
    wait_vmem();
    __syncthreads();  // level table and group g_begin ready
    for (int grp = g_begin; grp < g_end; ++grp) {
        const int buf = (grp - g_begin) & 1;
        if (grp + 1 < g_end) copy_group(grp + 1, buf ^ 1);
        if ((int64_t)(grp + 1) * C::GK > K)
            compute(buf, grp, std::true_type());
        else
            compute(buf, grp, std::false_type());
        wait_vmem();
        __syncthreads();  // group grp + 1 landed; every wave is done reading this buffer
    }

    // C[4 h + i][r] of tile t, block mb: weight row nw0 + 16 t + 4 h + i, activation row 16 mb + r
    const uint16_t* bias = reinterpret_cast<const uint16_t*>(g.bias);
#pragma unroll
    for (int t = 0; t < R; ++t)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int64_t m = 16 * mb + r;
            const int64_t nc = nw0 + 16 * t + 4 * h;
            if (m >= M || nc >= N) continue;  // N % 8 == 0: all four columns valid
            if (g.splits > 1) {
                *reinterpret_cast<float4*>(g.partial + (int64_t)z * M * N + m * N + nc) =
                    make_float4(acc[t][mb][0], acc[t][mb][1], acc[t][mb][2], acc[t][mb][3]);
            } else {
                float v[4] = {acc[t][mb][0], acc[t][mb][1], acc[t][mb][2], acc[t][mb][3]};
                if (bias) {  // 2-byte aligned: four 16-bit loads, issued together
                    uint16_t bb[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) bb[i] = bias[nc + i];
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] += Tr::to_f32(bb[i]);
                }
                uint2 pk;
                pk.x = Tr::pack2(v[0], v[1]);
                pk.y = Tr::pack2(v[2], v[3]);
                *reinterpret_cast<uint2*>(yo + m * N + nc) = pk;
            }
        }
}

// Small-M forward without a split reduction (up to 16 activation rows). A
// work-group owns 16 T weight rows (T MFMA tiles of 16 rows); a wave takes TW
// of them (TW = 1 or 2) and the 8 waves split the reduction into S = 8 TW / T
// slices: wave w takes tiles TW (w % (T / TW)) .. + TW - 1 and slice
// s = w / (T / TW), and in step j works on group j S + s (256 deep), so one
// step streams S consecutive groups (S x 128 contiguous bytes of every weight
// row). Operands reach LDS through lane-contiguous global -> LDS copies,
// double-buffered, one barrier per step; only the valid activation rows are
// copied (XR rows per slice; lanes past M use zero activations). The
// dequantization and MFMAs per group are those of k_gemv_fwd. At the end the
// slices' sums meet in LDS and the waves of slice 0 add them in slice order,
// then the rank-R LoRA term and the bias, and store: one launch, no fp32
// partials.
template <int T, int TW, int XR>
struct GkCfg {
    static constexpr int P = T / TW, S = 8 / P, ROWS = 16 * T;
    static constexpr int kLut = 256 * RW_LUT_COPIES * 8;
    static constexpr int kW = S * ROWS * 128;    // packed bytes of the step's S groups
    static constexpr int kA = S * ROWS * 4 * 4;  // absmax, up to 4 blocks per row and group
    static constexpr int kX = S * XR * 512;      // activations, XR rows per group
    static constexpr int kBuf = kW + kA + kX;
    static constexpr int kLds = kLut + 2 * kBuf;
    static_assert(T % TW == 0 && 8 % P == 0 && kLds <= 160 * 1024, "LDS");
    static_assert(S * XR * 32 <= 1024, "at most two activation copies per thread");
    static_assert(8 * TW * 64 * 16 <= kW, "the slice sums fit the weight buffer");
};

template <typename Tr, int T, int TW, int XR>
__global__ __launch_bounds__(512) void k_gemv_ks(GemmArgs g) {
    using C = GkCfg<T, TW, XR>;
    constexpr int S = C::S, ROWS = C::ROWS, P = C::P;
    constexpr int RS = S * ROWS;  // row-slices per step: 128 TW
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = (wave % P) * TW, s = wave / P;
    __shared__ __align__(16) uint8_t smem[C::kLds];
    float2* lut_all = reinterpret_cast<float2*>(smem);
    auto bw = [&](int b) { return reinterpret_cast<uint4*>(smem + C::kLut + b * C::kBuf); };  // [S][ROWS][8]
    auto ba = [&](int b) { return reinterpret_cast<float*>(smem + C::kLut + b * C::kBuf + C::kW); };
    auto bx = [&](int b) { return reinterpret_cast<uint4*>(smem + C::kLut + b * C::kBuf + C::kW + C::kA); };

    const int64_t K = g.K, N = g.N, M = g.M;
    const int bshift = 31 - __builtin_clz(g.blocksize);
    const int nfl = (GV_GK >> bshift) > 0 ? (GV_GK >> bshift) : 1;  // absmax per row per group
    const int64_t kblocks = K >> bshift;
    const int ngroups = (int)((K + GV_GK - 1) / GV_GK);
    const int steps = (ngroups + S - 1) / S;
    const int64_t n0 = (int64_t)blockIdx.x * ROWS;
    auto uniform = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane(v); };

    // copy sources, per thread. Packed weight: row-slice q = 16 TW wave + 8 i +
    // lane / 8 of the step's RS, 16-byte piece (lane % 8) ^ key(row).
    const uint8_t* wsrc[2 * TW];
    int wsl[2 * TW], wpiece[2 * TW];
#pragma unroll
    for (int i = 0; i < 2 * TW; ++i) {
        const int q = 16 * TW * wave + 8 * i + (lane >> 3), row = q % ROWS;
        wsl[i] = q / ROWS;
        wpiece[i] = (lane & 7) ^ ((row >> 1) & 7);
        const int64_t n = n0 + row < N ? n0 + row : N - 1;
        wsrc[i] = g.packed + n * (K / 2) + 16 * wpiece[i];
    }
    // absmax: thread tid copies entries e = tid + 512 i = (row-slice q) nfl + j
    // of RS nfl (whole waves: 128 TW nfl entries)
    const int acount = RS * nfl;
    const float* asrc[TW];
    int asl[TW], aj[TW];
#pragma unroll
    for (int i = 0; i < TW; ++i) {
        const int e = tid + 512 * i, q = (e < acount ? e : 0) / nfl;
        asl[i] = q / ROWS;
        aj[i] = e % nfl;
        const int64_t n = n0 + q % ROWS < N ? n0 + q % ROWS : N - 1;
        asrc[i] = g.absmax + n * kblocks;
    }
    // activations: piece p = tid + 512 i of S x XR x 32 (row xr of slice xs)
    const uint16_t* xsrc[2];
    int xsl[2], xpiece[2];
    bool xon[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = tid + 512 * i, xr = (p / 32) % XR;
        xsl[i] = p / (XR * 32);
        xon[i] = p < S * XR * 32 && xr < M;
        xpiece[i] = (p % 32) ^ (xr & 15);
        xsrc[i] = reinterpret_cast<const uint16_t*>(g.a) + (xr < M ? xr : 0) * K;
    }

    auto copy_step = [&](int j, int b) {
#pragma unroll
        for (int i = 0; i < 2 * TW; ++i) {
            int grp = j * S + wsl[i];
            grp = grp < ngroups ? grp : ngroups - 1;
            const int64_t off = (int64_t)grp * (GV_GK / 2);
            // bytes past the row (K % 256 != 0) read the row start instead
            const uint8_t* src = off + 16 * wpiece[i] < K / 2 ? wsrc[i] + off : wsrc[i] - 16 * wpiece[i];
            dma16(src, uniform(lds_offset(bw(b) + (16 * TW * wave + 8 * i) * 8)));
        }
#pragma unroll
        for (int i = 0; i < TW; ++i)
            if (tid + 512 * i < acount) {
                int grp = j * S + asl[i];
                grp = grp < ngroups ? grp : ngroups - 1;
                int64_t blk = (((int64_t)grp * GV_GK) >> bshift) + aj[i];
                blk = blk < kblocks ? blk : kblocks - 1;
                dma4(asrc[i] + blk, uniform((uint32_t)(size_t)((const __attribute__((address_space(3))) float*)(
                                        ba(b) + 512 * i + 64 * wave))));
            }
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (xon[i]) {
                int grp = j * S + xsl[i];
                grp = grp < ngroups ? grp : ngroups - 1;
                const int64_t k = (int64_t)grp * GV_GK + 8 * xpiece[i];
                dma16(xsrc[i] + (k < K ? k : 0), uniform(lds_offset(bx(b) + 512 * i + 64 * wave)));
            }
    };

    const int r = lane & 15, h = lane >> 4;
    const uint32_t copy_off = 8u * (uint32_t)(lane & 31);
    f32x4_t acc[TW];
#pragma unroll
    for (int u = 0; u < TW; ++u) acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int rx = r < XR ? r : 0;

    auto issue = [&](const uint4& qv, f32x2_t (&pp)[4][4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t word = q == 0 ? qv.x : q == 1 ? qv.y : q == 2 ? qv.z : qv.w;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t addr = __builtin_amdgcn_perm(copy_off, word, 0x0C0C0004u | ((uint32_t)b << 8));
                pp[q][b] = *(const __attribute__((address_space(3))) f32x2_t*)(size_t)addr;
            }
        }
    };
    // group j S + s of buffer b: items i = TW c + u (chunk c of tile t0 + u; k =
    // 128 c + 32 h + 0..31 on lane (r, h)); the table reads of item i + 1 are
    // written before item i's math, unfenced as in k_gemv_fwd
    // activation rows at or past M (never copied) only reach output columns
    // that are not stored, so they are read as they are; TAIL (the group that
    // reaches past K) zeroes the activations and scales of lanes past K
    auto compute = [&](int j, int b, auto tail_c) {
        constexpr bool TAIL = decltype(tail_c)::value;
        const int grp = j * S + s;
        const int64_t kg = (int64_t)grp * GV_GK;
        uint4 qv[2 * TW], xv[2][4];
        float av[2 * TW];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const bool ok = !TAIL || kg + 128 * c + 32 * h < K;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 v = bx(b)[(s * XR + rx) * 32 + ((16 * c + 4 * h + q) ^ r)];
                xv[c][q] = ok ? v : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < TW; ++u) {
                const int row = 16 * (t0 + u) + r, qrow = s * ROWS + row;
                qv[TW * c + u] = bw(b)[qrow * 8 + ((4 * c + h) ^ ((row >> 1) & 7))];
                const float a = ba(b)[qrow * nfl + ((128 * c + 32 * h) >> bshift)];
                av[TW * c + u] = ok ? a : 0.0f;
            }
        }
        f32x2_t p[2][4][4];
        issue(qv[0], p[0]);
#pragma unroll
        for (int i = 0; i < 2 * TW; ++i) {
            if (i + 1 < 2 * TW) issue(qv[i + 1], p[(i + 1) & 1]);
            const int c = i / TW, u = i % TW;
            const float a = av[i];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x2_t(&pq)[4] = p[i & 1][q];
                uint4 w;
                w.x = Tr::pack2(opaque(pq[0].x * a), opaque(pq[0].y * a));
                w.y = Tr::pack2(opaque(pq[1].x * a), opaque(pq[1].y * a));
                w.z = Tr::pack2(opaque(pq[2].x * a), opaque(pq[2].y * a));
                w.w = Tr::pack2(opaque(pq[3].x * a), opaque(pq[3].y * a));
                acc[u] = mfma16<Tr>(w, xv[c][q], acc[u]);
            }
        }
    };

    if (steps > 0) copy_step(0, 0);  // in flight while the level table is filled
    fill_lut_rw<512>(lut_all, tid);
    wait_vmem();
    __syncthreads();  // level table and step 0 ready
    for (int j = 0; j < steps; ++j) {
        const int b = j & 1;
        if (j + 1 < steps) copy_step(j + 1, b ^ 1);
        const int grp = j * S + s;
        if ((int64_t)(grp + 1) * GV_GK > K) {
            if (grp < ngroups) compute(j, b, std::true_type());
        } else {
            compute(j, b, std::false_type());
        }
        wait_vmem();
        __syncthreads();  // step j + 1 landed; every wave is done with buffer b
    }

    // the slices' sums meet in LDS (the weight buffer of buffer 0): entry
    // (slice, tile) of TW tiles per wave, 64 lanes
    float4* red = reinterpret_cast<float4*>(bw(0));
#pragma unroll
    for (int u = 0; u < TW; ++u)
        red[(s * T + t0 + u) * 64 + lane] = make_float4(acc[u][0], acc[u][1], acc[u][2], acc[u][3]);
    __syncthreads();
    if (s != 0) return;
    const int R = g.lora_rank;
    const uint16_t* bias = reinterpret_cast<const uint16_t*>(g.bias);
#pragma unroll
    for (int u = 0; u < TW; ++u) {
        float v[4] = {acc[u][0], acc[u][1], acc[u][2], acc[u][3]};
#pragma unroll
        for (int sl = 1; sl < S; ++sl) {
            const float4 o = red[(sl * T + t0 + u) * 64 + lane];
            v[0] += o.x;
            v[1] += o.y;
            v[2] += o.z;
            v[3] += o.w;
        }
        // C[4 h + i][r] of tile t0 + u: weight row n0 + 16 (t0 + u) + 4 h + i, activation row r
        const int64_t m = r, nc = n0 + 16 * (t0 + u) + 4 * h;
        if (m >= M || nc >= N) continue;  // N % 8 == 0: all four columns valid
        if (R > 0) {  // R % 16 == 0; T, L 16-byte aligned: 8 ranks per load
            const uint4* t8 =
                reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(g.lora_x) + m * R);
            const uint16_t* L = reinterpret_cast<const uint16_t*>(g.lora_w);
            float l[4] = {0.f, 0.f, 0.f, 0.f};
            for (int k8 = 0; k8 < R / 8; ++k8) {
                const uint4 tv = t8[k8];
                const uint32_t tw[4] = {tv.x, tv.y, tv.z, tv.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint4 lv = reinterpret_cast<const uint4*>(L + (nc + i) * R)[k8];
                    const uint32_t lw[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        l[i] += Tr::to_f32((uint16_t)(tw[q] & 0xFFFF)) * Tr::to_f32((uint16_t)(lw[q] & 0xFFFF));
                        l[i] += Tr::to_f32((uint16_t)(tw[q] >> 16)) * Tr::to_f32((uint16_t)(lw[q] >> 16));
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] += l[i];
        }
        if (bias) {
            uint16_t bb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) bb[i] = bias[nc + i];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] += Tr::to_f32(bb[i]);
        }
        uint2 pk;
        pk.x = Tr::pack2(v[0], v[1]);
        pk.y = Tr::pack2(v[2], v[3]);
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(g.out) + m * N + nc) = pk;
    }
}

// ----------------------------------------------------- small-M input gradient
// dX[M, K] = dY[M, N] . W[N, K] for M <= 64 rows, bound by dequantizing the
// streamed weight. A work-group owns 256 output columns k (128 bytes of every
// packed weight row) and one range of weight rows n (the reduction), walked in
// groups of GN rows (256, or 128 above 16 rows, whose larger dY buffers
// must fit); each range writes fp32 partials [split][m][k] that k_split_reduce
// sums (adding the LoRA term U . At^T). Wave w owns the columns [32 w, 32 w + 32)
// of the block: two 16-column tiles of v_mfma_f32_16x16x32 (weight side: 16
// columns x 32 rows n; dY side: 32 rows n x 16 activation rows, MB blocks of
// them), the two 8-byte halves of 16-byte chunk w of every packed row.
// Operands reach LDS through lane-contiguous global -> LDS copies,
// double-buffered, one barrier per group:
//  - packed weight: GN rows x 128 bytes, chunk q of row r in slot q ^ key(r);
//  - absmax: [column block][GN rows], dword copies of one row per lane;
//  - dY: M rows x GN n, piece p (8 values) of row m in slot p ^ (m % 16); rows
//    M .. XR - 1 are zeroed once and never copied.
// The weight-side operand needs 8 consecutive n of one column per lane: a
// ds_read_b64_tr_b4 of 16 rows x 16 columns, in which lane i of a 16-lane group
// points at 8 bytes of row i and lane c receives nibble c of the 16 rows, row r
// in nibble r. Nibble c is the low nibble of byte c / 2 for even c and packed
// NF4 keeps the even column in the high nibble, so lane c holds column c ^ 1
// (undone by the store). In 64-row subgroup u, lane group g reads rows
// 64 u + 16 g + 0..15; the first word (rows 0..7) feeds the tile's first MFMA
// and the second word (rows 8..15) its second, the dY operand taking the same
// rows (the assignment of rows to reduction slots is free when both operands
// agree). Each weight row has its own absmax, so a lane applies 16 per
// subgroup (four broadcast 16-byte reads). The dequantization is the register
// path of the other kernels: a perm-built level-table address per byte, an
// fp32 product per element, one rounding.
template <int MB>
struct GbCfg {
    static constexpr int KW = 256, GN = MB == 1 ? 256 : 128, XR = 16 * MB;
    static constexpr int XC = XR * (GN / 8) / 512;  // dY copies per wave and group
    static constexpr int NSUB = GN / 64;   // 64-row subgroups per group
    static constexpr int PR = GN / 8;      // 16-byte dY pieces per row and group
    static constexpr int kLut = 256 * RW_LUT_COPIES * 8;
    static constexpr int kW = GN * 128;    // packed rows of a group
    static constexpr int kA = 4 * GN * 4;  // absmax, up to 4 column blocks
    static constexpr int kX = XR * GN * 2; // dY rows of the group
    static constexpr int kBuf = kW + kA + kX;
    static constexpr int kLds = kLut + 2 * kBuf;
    static_assert(kLds <= 160 * 1024, "LDS");
    static_assert(XR * PR == 512 * XC && XC >= 1, "whole dY copies per wave and group");
    static_assert(PR >= 16 && PR <= 32 && (PR & (PR - 1)) == 0, "piece p ^ (m % 16) stays within the row");
};
constexpr int GB_MAX_M = 64;

template <typename Tr, int MB>
__global__ __launch_bounds__(512) void k_gemv_bwd(GemmArgs g, int groups_per_split) {
    using C = GbCfg<MB>;
    constexpr int GN = C::GN, NSUB = C::NSUB, PR = C::PR, NI = 2 * NSUB;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    __shared__ __align__(16) uint8_t smem[C::kLds];
    float2* lut_all = reinterpret_cast<float2*>(smem);
    auto bw = [&](int b) { return reinterpret_cast<uint4*>(smem + C::kLut + b * C::kBuf); };  // [GN][8]
    auto ba = [&](int b) { return reinterpret_cast<float*>(smem + C::kLut + b * C::kBuf + C::kW); };
    auto bx = [&](int b) { return reinterpret_cast<uint4*>(smem + C::kLut + b * C::kBuf + C::kW + C::kA); };

    const int64_t K = g.K, N = g.N, M = g.M;
    const int bshift = 31 - __builtin_clz(g.blocksize);
    const int64_t kblocks = K >> bshift;
    const int nbw = (C::KW >> bshift) > 0 ? (C::KW >> bshift) : 1;  // column blocks of the work-group
    const int ngroups = (int)((N + GN - 1) / GN);
    // tile T = z nb + x (column block x of range z). The hardware deals
    // consecutive work-groups to the 8 XCDs in turn, so work-group L runs tile
    // (L % 8) q + L / 8 of the 8 q launched: each XCD gets a contiguous run of
    // column blocks of one range, which share the absmax lines and dY rows in
    // its L2 (dealt round-robin, every absmax line went to all 8 XCDs).
    const int nb = (int)((K + C::KW - 1) / C::KW), splits = (ngroups + groups_per_split - 1) / groups_per_split;
    const int q8 = (int)(gridDim.x / 8);
    const int T = (int)(blockIdx.x % 8) * q8 + (int)(blockIdx.x / 8);
    if (T >= nb * splits) return;
    const int z = T / nb;
    const int g_begin = z * groups_per_split;
    const int g_end = g_begin + groups_per_split < ngroups ? g_begin + groups_per_split : ngroups;
    const int64_t k0 = (int64_t)(T % nb) * C::KW, kb0 = k0 >> bshift;
    const uint16_t* dy = reinterpret_cast<const uint16_t*>(g.a);
    auto uniform = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane(v); };

    // packed-weight copies: instruction NSUB wave + j covers rows 8 (NSUB wave + j) + 0..7;
    // the lane takes row 8 (NSUB wave + j) + lane / 8, chunk (lane % 8) ^ key(row)
    // (chunks past K re-read the row's last one: they feed unstored columns)
    int wrow[NSUB];
    int64_t wcol[NSUB];
#pragma unroll
    for (int j = 0; j < NSUB; ++j) {
        wrow[j] = 8 * (NSUB * wave + j) + (lane >> 3);
        const int64_t cb = k0 / 2 + 16 * ((lane & 7) ^ swz_key(wrow[j]));
        wcol[j] = cb + 16 <= K / 2 ? cb : K / 2 - 16;
    }
    // dY copies: copy j of wave w fills slots 512 j + 64 w + lane of the XR x PR
    // slots, i.e. slot lane % PR of row (512 j + 64 w + lane) / PR, piece
    // (lane % PR) ^ (row % 16), when the row exists
    int xm[C::XC], xp[C::XC];
    const uint16_t* xsrc[C::XC];
#pragma unroll
    for (int j = 0; j < C::XC; ++j) {
        xm[j] = (512 * j + 64 * wave + lane) / PR;
        xp[j] = (lane % PR) ^ (xm[j] & 15);
        xsrc[j] = dy + (xm[j] < M ? xm[j] : 0) * N + 8 * xp[j];
    }

    auto copy_group = [&](int grp, int b) {
        const int64_t n0 = (int64_t)grp * GN;
#pragma unroll
        for (int j = 0; j < NSUB; ++j) {
            const int64_t n = n0 + wrow[j] < N ? n0 + wrow[j] : N - 1;
            dma16(g.packed + n * (K / 2) + wcol[j], uniform(lds_offset(bw(b) + (NSUB * wave + j) * 64)));
        }
        // absmax: instruction i = wave + 8 j (< NSUB nbw) covers block i / NSUB,
        // rows 64 (i % NSUB) + lane
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = wave + 8 * j;
            if (i < NSUB * nbw) {
                const int64_t r = n0 + 64 * (i % NSUB) + lane;
                const int64_t n = r < N ? r : N - 1;
                const int64_t kb = kb0 + i / NSUB < kblocks ? kb0 + i / NSUB : kblocks - 1;
                dma4(g.absmax + n * kblocks + kb,
                     uniform((uint32_t)(size_t)((const __attribute__((address_space(3))) float*)(ba(b) + 64 * i))));
            }
        }
#pragma unroll
        for (int j = 0; j < C::XC; ++j)
            if (xm[j] < M)
                dma16(xsrc[j] + (n0 + 8 * xp[j] < N ? n0 : -8 * xp[j]), uniform(lds_offset(bx(b) + 512 * j + 64 * wave)));
    };

    const int c = lane & 15, gq = lane >> 4;
    const uint32_t copy_off = 8u * (uint32_t)(lane & 31);
    // transposed read of subgroup u, tile t: row 16 gq + c of the subgroup,
    // chunk wave (slot wave ^ key(row), key(row) = c / 2 here), half t
    const uint32_t tr_lane = 128u * (uint32_t)(16 * gq + c) + 16u * (uint32_t)(wave ^ (c >> 1));
    const int wblk = (int)(((k0 + 32 * wave) >> bshift) - kb0);  // this wave's column block (< nbw)
    f32x4_t acc[2][MB];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[t][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // table reads of one transposed read: word wd, byte bb (rows 8 wd + 2 bb, + 1)
    auto issue = [&](const v2i32_t& v, f32x2_t (&pp)[2][4]) {
#pragma unroll
        for (int wd = 0; wd < 2; ++wd) {
            const uint32_t word = (uint32_t)(wd ? v.y : v.x);
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                const uint32_t addr = __builtin_amdgcn_perm(copy_off, word, 0x0C0C0004u | ((uint32_t)bb << 8));
                pp[wd][bb] = *(const __attribute__((address_space(3))) f32x2_t*)(size_t)addr;
            }
        }
    };
    // one group: items i = 2 u + t; the table reads of item i + 1 are written
    // before item i's math, with no scheduling fence between items (1-7 %
    // faster than fenced items). TAIL (the group reaching past N) zeroes the
    // absmax and dY of subgroups past N.
    auto compute = [&](int grp, int b, auto tail_c) {
        constexpr bool TAIL = decltype(tail_c)::value;
        const int64_t n0 = (int64_t)grp * GN;
        const uint32_t wt = lds_offset(bw(b)) + tr_lane;
        v2i32_t tr[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i)
            tr[i] = __builtin_amdgcn_ds_read_tr4_b64_v2i32(
                (__attribute__((address_space(3))) v2i32_t*)(size_t)(wt + 8192u * (uint32_t)(i >> 1) +
                                                                     8u * (uint32_t)(i & 1)));
        f32x2_t p[2][2][4];
        f32x4_t av[4];
        uint4 xv[2][MB];
        issue(tr[0], p[0]);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int u = i >> 1, t = i & 1;
            if (t == 0) {
                const bool ok = !TAIL || n0 + 64 * u < N;
                const float* ap = ba(b) + wblk * GN + 64 * u + 16 * gq;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(ap + 4 * q);
                    av[q] = ok ? a : f32x4_t{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) {
                        const uint4 v = bx(b)[(16 * mb + c) * PR + ((8 * u + 2 * gq + s) ^ c)];
                        xv[s][mb] = ok ? v : make_uint4(0, 0, 0, 0);
                    }
            }
            if (i + 1 < NI) issue(tr[i + 1], p[(i + 1) & 1]);
#pragma unroll
            for (int wd = 0; wd < 2; ++wd) {
                // byte bb: row 8 wd + 2 bb in the low nibble (.y), row 8 wd + 2 bb + 1 in the high (.x)
                const f32x2_t(&pq)[4] = p[i & 1][wd];
                const f32x4_t a0 = av[2 * wd], a1 = av[2 * wd + 1];
                uint4 w;
                w.x = Tr::pack2(opaque(pq[0].y * a0[0]), opaque(pq[0].x * a0[1]));
                w.y = Tr::pack2(opaque(pq[1].y * a0[2]), opaque(pq[1].x * a0[3]));
                w.z = Tr::pack2(opaque(pq[2].y * a1[0]), opaque(pq[2].x * a1[1]));
                w.w = Tr::pack2(opaque(pq[3].y * a1[2]), opaque(pq[3].x * a1[3]));
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) acc[t][mb] = mfma16<Tr>(w, xv[wd][mb], acc[t][mb]);
            }
        }
    };

    if (g_begin < g_end) copy_group(g_begin, 0);  // in flight while the tables are set up
    for (int i = tid; i < 2 * C::XR * PR; i += 512) {  // dY rows M .. XR - 1 of both buffers stay zero
        const int s = i % (C::XR * PR);
        if (s / PR >= M) bx(i / (C::XR * PR))[s] = make_uint4(0, 0, 0, 0);
    }
    fill_lut_rw<512>(lut_all, tid);
    wait_vmem();
    __syncthreads();  // level table, zero rows and group g_begin ready
    for (int grp = g_begin; grp < g_end; ++grp) {
        const int b = (grp - g_begin) & 1;
        if (grp + 1 < g_end) copy_group(grp + 1, b ^ 1);
        if ((int64_t)(grp + 1) * GN > N)
            compute(grp, b, std::true_type());
        else
            compute(grp, b, std::false_type());
        wait_vmem();
        __syncthreads();  // group grp + 1 landed; every wave is done with buffer b
    }

    // D[i][j] of tile t, block mb sits in lane j + 16 (i / 4), element i % 4:
    // activation row 16 mb + j (j = lane % 16), A row i = 4 gq + e, i.e. column
    // 16 t + ((4 gq + e) ^ 1) of this wave's 32
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = 16 * mb + (lane & 15);
        if (m >= M) continue;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int64_t col = k0 + 32 * wave + 16 * t + 4 * gq;
            if (col < K)  // K % 64 == 0: all four columns valid
                *reinterpret_cast<float4*>(g.partial + ((int64_t)z * M + m) * K + col) =
                    make_float4(acc[t][mb][1], acc[t][mb][0], acc[t][mb][3], acc[t][mb][2]);
        }
    }
}

// Sum of the split partials [splits][rows][cols] (+ bias) (+ T[row] . L[col]
// over R ranks, when R > 0), one rounding; four columns per lane (cols % 4 == 0).
template <typename Tr>
__global__ __launch_bounds__(256) void k_split_reduce(const float* __restrict__ partial, int splits, int64_t rows,
                                                      int64_t cols, const uint16_t* __restrict__ bias,
                                                      const uint16_t* __restrict__ T, const uint16_t* __restrict__ L,
                                                      int R, uint16_t* __restrict__ out) {
    const int64_t total = rows * (cols / 4), plane = rows * cols;
    for (int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; v < total; v += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = v * 4;
        // partials summed in split order; four loads in flight at a time
        float4 acc = *reinterpret_cast<const float4*>(partial + e);
        int z = 1;
        for (; z + 4 <= splits; z += 4) {
            float4 p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = *reinterpret_cast<const float4*>(partial + (z + i) * plane + e);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc.x += p[i].x;
                acc.y += p[i].y;
                acc.z += p[i].z;
                acc.w += p[i].w;
            }
        }
        for (; z < splits; ++z) {
            const float4 p = *reinterpret_cast<const float4*>(partial + z * plane + e);
            acc.x += p.x;
            acc.y += p.y;
            acc.z += p.z;
            acc.w += p.w;
        }
        if (R > 0) {  // R % 16 == 0; T, L 16-byte aligned: 8 ranks per load
            const int64_t row = e / cols, c = e % cols;
            const uint4* t8 = reinterpret_cast<const uint4*>(T + row * R);
            float l[4] = {0.f, 0.f, 0.f, 0.f};
            for (int k8 = 0; k8 < R / 8; ++k8) {
                const uint4 tv = t8[k8];
                uint4 lv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) lv[i] = reinterpret_cast<const uint4*>(L + (c + i) * R)[k8];
                const uint32_t tw[4] = {tv.x, tv.y, tv.z, tv.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t lw[4] = {lv[i].x, lv[i].y, lv[i].z, lv[i].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        l[i] += Tr::to_f32((uint16_t)(tw[j] & 0xFFFF)) * Tr::to_f32((uint16_t)(lw[j] & 0xFFFF));
                        l[i] += Tr::to_f32((uint16_t)(tw[j] >> 16)) * Tr::to_f32((uint16_t)(lw[j] >> 16));
                    }
                }
            }
            acc.x += l[0];
            acc.y += l[1];
            acc.z += l[2];
            acc.w += l[3];
        }
        if (bias) {
            const int64_t c = e % cols;
            acc.x += Tr::to_f32(bias[c]);
            acc.y += Tr::to_f32(bias[c + 1]);
            acc.z += Tr::to_f32(bias[c + 2]);
            acc.w += Tr::to_f32(bias[c + 3]);
        }
        uint2 pk;
        pk.x = Tr::pack2(acc.x, acc.y);
        pk.y = Tr::pack2(acc.z, acc.w);
        *reinterpret_cast<uint2*>(out + e) = pk;
    }
}

// lora: add the rank-R term here (the small-M forward leaves it to the reduce)
int launch_split_reduce(const GemmArgs& g, int64_t cols, const void* bias, int dtype, hipStream_t stream,
                        bool lora = false) {
    const int64_t items = g.M * (cols / 4);
    if (items == 0) return STM_OK;
    const int64_t blocks = (items + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 16384 ? blocks : 16384);
    const int R = lora ? g.lora_rank : 0;
    const uint16_t* T = R ? (const uint16_t*)g.lora_x : nullptr;
    const uint16_t* L = R ? (const uint16_t*)g.lora_w : nullptr;
    if (dtype == STM_BF16)
        hipLaunchKernelGGL(k_split_reduce<BF16>, dim3(grid), dim3(256), 0, stream, g.partial, g.splits, g.M, cols,
                           (const uint16_t*)bias, T, L, R, (uint16_t*)g.out);
    else
        hipLaunchKernelGGL(k_split_reduce<F16>, dim3(grid), dim3(256), 0, stream, g.partial, g.splits, g.M, cols,
                           (const uint16_t*)bias, T, L, R, (uint16_t*)g.out);
    return check_launch("gemm split reduce");
}


#ifndef STM_GEMV_MAX_M
#define STM_GEMV_MAX_M 64
#endif

#ifndef STM_GEMV_T_LAT
#define STM_GEMV_T_LAT 3.0  // small-M input gradient: fixed cost of a work-group, in groups
#endif

// Small-M forward plan: layout (activation blocks MB, group depth) and
// reduction ranges minimising an estimate fitted to forced range counts over
// ten or eleven weight shapes (N, K from 1024 to 28672) at three row counts
// per layout, in µs: a launch term, a cost per round of work-groups (one per
// CU) and per group and round, and with a split a reduce term per launch, per
// MB of fp32 partials and per range. At 17-32 rows both
// MB = 2 layouts are estimated and the faster taken: 192 weight rows over
// groups of 256 (6 waves) wins at N <= 6144 with K >= 2048, 256 rows over
// groups of 128 (8 waves) at larger N or short K (e.g. [28672,4096]
// 37.7 -> 29.8 us, [3072,1024] 13.4 -> 10.4 us at M = 17).
struct GemvFit {
    double launch, round, group, split, per_mb, per_range;
};
constexpr GemvFit kGv1{4.18, 0.85, 1.69, 2.32, 0.52, 0.132};       // MB = 1, groups of 256 (2 % rms)
constexpr GemvFit kGv2Deep{4.97, 1.23, 1.91, 1.76, 0.47, 0.079};   // MB = 2, groups of 256 (7 % rms)
constexpr GemvFit kGv2Short{4.34, 1.09, 1.10, 2.91, 0.41, 0.072};  // MB = 2, groups of 128 (3 % rms)
constexpr GemvFit kGv4{5.15, 0.86, 1.61, 2.87, 0.38, 0.077};       // MB = 4, groups of 128 (3 % rms)

struct GemvPlan {
    int mb = 1, gk = 256, rows = 256, splits = 1;
    double est = 0.0;
};

GemvPlan gemv_ranges(int mb, int gk, int rows, const GemvFit& fit, int64_t M, int64_t N, int64_t K) {
    GemvPlan p;
    p.mb = mb, p.gk = gk, p.rows = rows;
    const int64_t blocks = (N + rows - 1) / rows, groups = (K + gk - 1) / gk;
    double best_t = 1e30;
    for (int64_t sp = 1; sp <= (groups > 1 ? groups : 1) && sp <= 64; ++sp) {
        const int64_t gps = groups > 0 ? (groups + sp - 1) / sp : 0;
        const int64_t spe = gps > 0 ? (groups + gps - 1) / gps : 1;
        const int64_t rounds = (blocks * spe + 255) / 256;
        const double t = fit.launch + (double)rounds * (fit.round + fit.group * (double)gps) +
                         (spe > 1 ? fit.split + fit.per_mb * 1e-6 * (double)(spe * M * N * 4) +
                                        fit.per_range * (double)spe
                                  : 0.0);
        if (t < best_t - 1e-9) best_t = t, p.splits = (int)spe;
    }
    p.est = best_t;
    return p;
}

GemvPlan gemv_plan(int64_t M, int64_t N, int64_t K) {
    if (M <= 16) return gemv_ranges(1, 256, GvCfg<1, 256>::ROWS, kGv1, M, N, K);
    if (M > 32 && M <= 48) return gemv_ranges(3, 128, GvCfg<3, 128>::ROWS, kGv4, M, N, K);
    if (M > 32) return gemv_ranges(4, 128, GvCfg<4, 128>::ROWS, kGv4, M, N, K);
    const GemvPlan deep = gemv_ranges(2, 256, GvCfg<2, 256>::ROWS, kGv2Deep, M, N, K);
    const GemvPlan shrt = gemv_ranges(2, 128, GvCfg<2, 128>::ROWS, kGv2Short, M, N, K);
    return shrt.est < deep.est ? shrt : deep;
}

bool use_gemv(int64_t M, int num_groups) { return num_groups == 1 && M > 0 && M <= STM_GEMV_MAX_M; }

int launch_gemv_fwd(GemmArgs g, const GemvPlan& p, int dtype, hipStream_t stream) {
    const int ngroups = (int)((g.K + p.gk - 1) / p.gk);
    const int gps = (ngroups + p.splits - 1) / p.splits;
    const int splits = gps ? (ngroups + gps - 1) / gps : 1;  // every range non-empty (K = 0: one empty range)
    g.splits = splits;
    dim3 grid((unsigned)((g.N + p.rows - 1) / p.rows), (unsigned)splits);
#define STM_GV_LAUNCH(MB, GK)                                                                    \
    {                                                                                            \
        static_assert(GvCfg<MB, GK>::ROWS > 0, "config");                                        \
        if (p.rows != GvCfg<MB, GK>::ROWS) return set_error(STM_ERR_INVALID, "gemv plan rows"); \
        dim3 block(64 * GvCfg<MB, GK>::WAVES);                                                   \
        if (dtype == STM_BF16)                                                                   \
            hipLaunchKernelGGL((k_gemv_fwd<BF16, MB, GK>), grid, block, 0, stream, g, gps);      \
        else                                                                                     \
            hipLaunchKernelGGL((k_gemv_fwd<F16, MB, GK>), grid, block, 0, stream, g, gps);       \
    }
    if (p.mb == 1 && p.gk == 256 && g.M <= 16)
        STM_GV_LAUNCH(1, 256)
    else if (p.mb == 2 && p.gk == 256 && g.M <= 32)
        STM_GV_LAUNCH(2, 256)
    else if (p.mb == 2 && p.gk == 128 && g.M <= 32)
        STM_GV_LAUNCH(2, 128)
    else if (p.mb == 3 && p.gk == 128 && g.M <= 48)
        STM_GV_LAUNCH(3, 128)
    else if (p.mb == 4 && p.gk == 128 && g.M <= 64)
        STM_GV_LAUNCH(4, 128)
    else
        return set_error(STM_ERR_INVALID, "gemm_fwd: small-M plan MB %d, groups of %d for %lld rows", p.mb, p.gk,
                         (long long)g.M);
#undef STM_GV_LAUNCH
    int rc = check_launch("gemm_fwd (small M)");
    if (rc != STM_OK || g.splits == 1) return rc;
    return launch_split_reduce(g, g.N, g.bias, dtype, stream, true);
}

#ifndef STM_PERSISTENT
#define STM_PERSISTENT 1
#endif

// Compute units of the current device (cached per device): the work-group count
// of a persistent launch, one work-group per CU (the kernels' LDS allows one).
int device_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

// 1-D grid over the work items (tile, group, split): all of them, or one
// work-group per CU looping over them.
dim3 work_grid(int64_t work) {
    const int64_t cap = STM_PERSISTENT ? (int64_t)device_cus() : work;
    return dim3((unsigned)(work < cap ? work : cap));
}

template <int BM, int BN, int WM, int WN>
int launch_fwd_cfg(const GemmArgs& g, int dtype, hipStream_t stream) {
    const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    if (tiles == 0) return STM_OK;
    const int64_t work = tiles * g.num_groups * g.splits;
    if (work > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "gemm_fwd: grid too large");
    dim3 grid = work_grid(work), block(WM * WN * 64);
    if (dtype == STM_BF16)
        hipLaunchKernelGGL((k_gemm_fwd<BF16, BM, BN, WM, WN>), grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL((k_gemm_fwd<F16, BM, BN, WM, WN>), grid, block, 0, stream, g);
    return check_launch("gemm_fwd");
}

template <int BM, int BN, int WM, int WN>
int launch_bwd_cfg(const GemmArgs& g, int dtype, hipStream_t stream) {
    const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.K + BN - 1) / BN);
    if (tiles == 0) return STM_OK;
    const int64_t work = tiles * g.num_groups * g.splits;
    if (work > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "gemm_bwd_dx: grid too large");
    dim3 grid = work_grid(work), block(WM * WN * 64);
    if (dtype == STM_BF16)
        hipLaunchKernelGGL((k_gemm_bwd<BF16, BM, BN, WM, WN>), grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL((k_gemm_bwd<F16, BM, BN, WM, WN>), grid, block, 0, stream, g);
    return check_launch("gemm_bwd_dx");
}

// The register-weight forward (k_gemm_fwd_rw) replaces the 256 x 256 LDS-weight
// forward for unsplit launches, single-matrix and grouped: measured on MI355X
// 7-10 % faster at M = 512 and 8192 on the 14336 x 4096 and 4096 x 14336
// weights and 5 % on a 128-expert bank (1536 x 2048 and 2048 x 768 experts,
// ~512 rows each). Split launches (small M) keep the LDS-weight kernels.
// STM_FWD_RW_WM = 2 (eight waves, 128 x 64 wave tiles, the dequantization done
// twice) measured 14 % slower.
#ifndef STM_FWD_RW
#define STM_FWD_RW 1
#endif

#ifndef STM_BWD_RW
#define STM_BWD_RW 1
#endif

// k_gemm_bwd_rw: 32-bit offsets for dY [M, N], the packed weight, absmax and dX [M, K].
bool rw_offsets_fit_bwd(const GemmArgs& g) {
    const int64_t lim = (int64_t)1 << 32;
    return g.M * g.N * 2 < lim && g.N * g.K / 2 < lim && g.N * g.K / g.blocksize < lim && g.M * g.K < lim / 2;
}

// k_gemm_fwd_rw addresses activations, packed weights and absmax of one group
// with 32-bit offsets from uniform bases.
bool rw_offsets_fit(const GemmArgs& g) {
    const int64_t lim = (int64_t)1 << 32;
    return g.M * g.K * 2 < lim && g.N * g.K / 2 < lim && g.N * g.K / g.blocksize < lim && g.M * g.N < lim / 2;
}

#ifndef STM_FWD_RW_WM
#define STM_FWD_RW_WM 1
#endif

template <int BM>
int launch_bwd_rw(const GemmArgs& g, int dtype, hipStream_t stream) {
    const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.K + 255) / 256);
    if (tiles == 0) return STM_OK;
    const int64_t work = tiles * g.num_groups * g.splits;
    if (work > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "gemm_bwd_dx: grid too large");
    dim3 grid = work_grid(work), block(256);
    if (dtype == STM_BF16)
        hipLaunchKernelGGL((k_gemm_bwd_rw<BF16, BM>), grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL((k_gemm_bwd_rw<F16, BM>), grid, block, 0, stream, g);
    return check_launch("gemm_bwd_dx");
}

int launch_fwd_r8(const GemmArgs& g, int dtype, hipStream_t stream) {
    const int64_t tiles = ((g.M + 255) / 256) * ((g.N + 255) / 256);
    if (tiles == 0) return STM_OK;
    const int64_t work = tiles * g.num_groups * g.splits;
    if (work > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "gemm_fwd: grid too large");
    dim3 grid = work_grid(work), block(512);
    if (dtype == STM_BF16)
        hipLaunchKernelGGL((k_gemm_fwd_r8<BF16>), grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL((k_gemm_fwd_r8<F16>), grid, block, 0, stream, g);
    return check_launch("gemm_fwd");
}

template <int BM, int WM>
int launch_fwd_rw(const GemmArgs& g, int dtype, hipStream_t stream) {
    const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + 255) / 256);
    if (tiles == 0) return STM_OK;
    const int64_t work = tiles * g.num_groups * g.splits;
    if (work > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "gemm_fwd: grid too large");
    dim3 grid = work_grid(work), block(256 * WM);
    if (dtype == STM_BF16)
        hipLaunchKernelGGL((k_gemm_fwd_rw<BF16, BM, WM>), grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL((k_gemm_fwd_rw<F16, BM, WM>), grid, block, 0, stream, g);
    return check_launch("gemm_fwd");
}

}  // namespace

namespace {

// Tile shape and split count of a problem: `cols` = output columns (N forward,
// K input gradient), `red` = reduction length (K forward, N input gradient).
// Both tile shapes run one work-group per CU (LDS), so a launch runs in waves
// of 256 work-groups (MI355X's CU count). Estimated time of a choice:
//   waves(tiles * splits) * (steps_per_split * t_step + t_wave) + reduce,
// t_step = time of one 64-deep step of one wave of tiles, measured at
// M = 2048..8192 on the 14336 x 4096 and 4096 x 14336 weights (forward: 2.0 us
// big tile with the register-weight kernel, 2.2 us with the LDS-weight kernel,
// 0.8 us 128 x 128; input gradient: 1.85 us, 2.45 us, 1.35 us), t_wave = 8 us of
// per-tile prologue and epilogue, reduce = the fp32 partials written and read
// once at 5 TB/s plus 4 us. Splits: at most 16, at least 8 steps each; grouped
// launches never split.
constexpr int kCUs = 256;

// Tile kinds: kBig = 256 x 256 (register-weight or LDS-weight kernel), kSmall =
// 128 x 128 (LDS-weight), kMid = 128 rows x 256 columns (register-weight, unsplit).
enum TileKind { kBig = 0, kSmall = 1, kMid = 2, kBig8 = 3 };

struct Plan {
    int kind;
    int64_t tiles;
    int splits;
};

double plan_cost(int64_t tiles, int64_t steps, int sp, double t_step, int64_t M, int64_t cols) {
    const int64_t waves = (tiles * sp + kCUs - 1) / kCUs;
    const int64_t per = (steps + sp - 1) / sp;
    double t = (double)waves * ((double)per * t_step + 8.0);
    if (sp > 1) t += ((double)sp * M * cols * 8.0 + (double)M * cols * 2.0) / 5.0e6 + 4.0;  // us
    return t;
}

// The 128 x 256 register-weight tile (kMid) as a cost-model choice (unsplit
// only). Input gradient: measured at M = 512..4096 on the 14336 x 4096 and
// 4096 x 14336 weights it is 0-12 % faster than the choices without it.
// Forward: it pays only where its tiles fill the GPU and the big tiles do not
// (M = 4096 on W [2048, 1024]: 32.9 us against 40.6); the per-step time is
// calibrated with every CU busy (1.55 us; 1.2-1.3 us on a half-empty GPU), so
// the model does not pick it on the 8B-class weights at M = 256..2048, where
// it measured -3..+5 %. Input gradient per step 1.1 us.
#ifndef STM_MID_TILE
#define STM_MID_TILE 1
#endif
#ifndef STM_T_MID_FWD
#define STM_T_MID_FWD 1.55  // per step with every CU busy (1.2-1.3 on a half-empty GPU)
#endif
// The forward's per-step time when its 128 x 256 tiles fill less than one
// round of the CUs. Measured with it on the shapes whose plan it flips from
// the split 256 x 256 tile to the unsplit 128 x 256 tile, µs before -> after:
// W [14336,4096] at M = 320 / 384 / 448: 87.9 / 85.0 / 86.0 -> 74.3 / 70.7 /
// 74.0; [8192,4096] at M = 640 / 768: 79.1 / 81.8 -> 69.6 / 70.5; [4096,4096]
// at M = 1408 / 1536: 80.2 / 81.5 -> 69.3 / 70.3; [5632,2048] at M = 704:
// 45.4 -> 39.0; [2048,5632] at M = 3072: 101.7 -> 93.2.
#ifndef STM_T_MID_FWD_PART
#define STM_T_MID_FWD_PART 1.25
#endif
#ifndef STM_T_MID_BWD
#define STM_T_MID_BWD 1.1
#endif
// Forward planner calibration, re-measured with the current kernels (auto
// plans, µs before -> after): the 128 x 128 tile's per-step time is 0.95 µs
// (0.8 before) and forward splits stop at 8 ranges (16 before: the model's
// 16-range plans measured slower). W [4096,4096] at M = 640: 58.1 -> 51.1;
// [6144,4096] at M = 384 / 512: 57.7 / 57.2 -> 50.7 / 54.1; [3072,4096] at
// M = 768 / 1024: 57.0 / 57.1 -> 48.1 / 54.2; K = 1024 shapes 2-5 % faster;
// no measured shape slower (19 shapes, M = 64-1024).
#ifndef STM_FWD_MAX_SPLIT
#define STM_FWD_MAX_SPLIT 8
#endif
#ifndef STM_T_SMALL_FWD
#define STM_T_SMALL_FWD 0.95
#endif
#ifndef STM_BWD_MID_MAX_STEPS
#define STM_BWD_MID_MAX_STEPS 48
#endif

// Whether a 256 x 256 launch of `splits` ranges over `steps` reduction steps runs
// the register-weight kernel. Measured on MI355X: unsplit always wins; split, the
// input gradient wins with at most 4 ranges of at least STM_RW_SPLIT_MIN_STEPS
// steps and loses with more, shorter ranges (+11..+41 % at 7..16 ranges of
// 14..32 steps); the split forward loses (+4..+20 %).
// Shortest range a split input gradient gives the register-weight kernel
// (shorter ranges take the LDS-weight kernel). Re-measured with the current
// kernels, auto plans, µs 32 -> 64: W [14336,4096] at M = 768 / 1024 142.5 /
// 171.5 -> 122.3 / 140.3; [6144,4096] at M = 1024 110.2 -> 85.9; [11008,4096]
// at M = 768 / 1024 123.6 / 152.6 -> 102.4 / 124.4; 14 other shapes unchanged.
#ifndef STM_RW_SPLIT_MIN_STEPS
#define STM_RW_SPLIT_MIN_STEPS 64
#endif
bool rw_split_ok(bool backward, int splits, int64_t steps) {
    if (splits <= 1) return true;
    return backward && splits <= 4 && (steps + splits - 1) / splits >= STM_RW_SPLIT_MIN_STEPS;
}

// Tile restriction: -1 = cost model, else one TileKind (tests use it to reach
// each kernel). Starts from STRATUM_NF4_GEMM_TILE = "big", "mid", "small" or
// "big8", read once when the library loads; stm_nf4_gemm_set_tile changes it.
int tile_from_env() {
    const char* v = getenv("STRATUM_NF4_GEMM_TILE");
    if (!v) return -1;
    if (strcmp(v, "big") == 0) return kBig;
    if (strcmp(v, "small") == 0) return kSmall;
    if (strcmp(v, "mid") == 0) return kMid;
    if (strcmp(v, "big8") == 0) return kBig8;
    return -1;
}

std::atomic<int> g_tile_only{tile_from_env()};

int tile_override() { return g_tile_only.load(std::memory_order_relaxed); }

Plan plan(int64_t M, int64_t cols, int64_t red, bool backward, int num_groups) {
    const int64_t bm = backward ? STM_BWD_BM : STM_FWD_BM, bn = backward ? STM_BWD_BN : STM_FWD_BN;
    const int64_t big_tiles = ((M + bm - 1) / bm) * ((cols + bn - 1) / bn) * num_groups;
    const int64_t small_tiles = ((M + 127) / 128) * ((cols + 127) / 128) * num_groups;
    const int64_t mid_tiles = ((M + 127) / 128) * ((cols + 255) / 256) * num_groups;
    const int64_t steps = red / BK;
    // big tiles run the register-weight kernels when unsplit, and for the input
    // gradient also when split into ranges of >= 32 steps (rw_split_ok)
    const double t_big_rw = backward ? 1.85 : 2.0, t_big = backward ? 2.45 : 2.2,
                 t_small = backward ? 1.35 : STM_T_SMALL_FWD;
    // (the input gradient's 128 x 256 tile gains nothing comparable on a part of
    // the CUs: the same change there measured -14 .. +9 % by shape)
    const double t_mid = backward ? STM_T_MID_BWD : (mid_tiles < kCUs ? STM_T_MID_FWD_PART : STM_T_MID_FWD);
    int max_sp = 1;
    if (num_groups == 1) {
        const int64_t by_steps = steps / 8;
        max_sp = (int)(by_steps < 16 ? (by_steps > 1 ? by_steps : 1) : 16);
        if (!backward && max_sp > STM_FWD_MAX_SPLIT) max_sp = STM_FWD_MAX_SPLIT;
    }
    const int only = tile_override();
    // Input gradient: the unsplit 128 x 256 tile when its tiles fill 1/4 to one
    // round of the CUs and the reduction is at most 48 steps (weights of up to
    // 3072 rows). The cost model favours split 256 x 256 launches there, which
    // measured slower, µs: W [2048,1024] at M = 2048 41.3 -> 35.6, [2048,2048]
    // at M = 1024 41.5 -> 35.8, [3072,1024] at M = 2048 50.2 -> 49.1, the other
    // such shapes within 1 %. At 88-96 steps the same rule measured -7 .. +43 %
    // ([5632,2048], [6144,1024], [6144,4096]), so longer reductions keep the model.
    if (STM_MID_TILE && backward && only < 0 && num_groups == 1 && mid_tiles >= kCUs / 4 && mid_tiles <= kCUs &&
        steps <= STM_BWD_MID_MAX_STEPS)
        return Plan{kMid, mid_tiles, 1};
    Plan best{only < 0 ? (int)kBig : only, only == kSmall ? small_tiles : only == kMid ? mid_tiles : big_tiles, 1};
    double best_t = 1e300;
    for (int sp = 1; sp <= max_sp; ++sp) {
        const double tb = plan_cost(big_tiles, steps, sp, rw_split_ok(backward, sp, steps) ? t_big_rw : t_big, M, cols);
        if ((only < 0 || only == kBig) && tb < best_t) {
            best_t = tb;
            best = Plan{kBig, big_tiles, sp};
        }
        const double ts = plan_cost(small_tiles, steps, sp, t_small, M, cols);
        if ((only < 0 || only == kSmall) && ts < best_t) {
            best_t = ts;
            best = Plan{kSmall, small_tiles, sp};
        }
        if (sp == 1 && (STM_MID_TILE || only == kMid)) {
            const double tm = plan_cost(mid_tiles, steps, 1, t_mid, M, cols);
            if ((only < 0 || only == kMid) && tm < best_t) {
                best_t = tm;
                best = Plan{kMid, mid_tiles, 1};
            }
        }
    }
    return best;
}

}  // namespace

// Cost of an expert's rows in units of one 256-row item of the grouped
// forward. 256-row tiles: one unit per full tile; the last, partial tile runs
// as a short item when it holds at most 64 or 128 rows (its MFMAs cut to a
// quarter or half, its weight work and fixed cost not). 192-row tiles: 0.81
// each (three quarters of the rows, 8 % dearer per row: the weight is
// dequantized for fewer rows). Measured on the 128-expert bank with 454-569
// rows per expert: 256-row tiles 462 us (gate/up) and 278 us (down) against
// 488 and 282 with 192-row tiles.
double grouped_cost(int64_t r, int bm) {
    if (r <= 0) return 0.0;
    if (bm == 192) return 0.81 * (double)((r + 191) / 192);
    const int64_t rem = r % 256;
    const double last = rem == 0 ? 0.0 : rem <= 64 ? 0.45 : rem <= 128 ? 0.6 : 1.0;
    return (double)(r / 256) + last;
}

int grouped_tile_rows(const int32_t* offsets, int num_experts) {
    double c256 = 0.0, c192 = 0.0;
    for (int e = 0; e < num_experts; ++e) {
        const int64_t r = (int64_t)offsets[e + 1] - offsets[e];
        c256 += grouped_cost(r, 256);
        c192 += grouped_cost(r, 192);
    }
    return c192 < c256 ? 192 : 256;
}

int set_gemm_tile(int kind) {
    return g_tile_only.exchange(kind >= kBig && kind <= kBig8 ? kind : -1, std::memory_order_relaxed);
}

int gemm_splits(int64_t M, int64_t N, int64_t K, bool backward, int num_groups) {
    return backward ? plan(M, K, N, true, num_groups).splits : plan(M, N, K, false, num_groups).splits;
}

int gemv_ks_tiles(int64_t M, int64_t N, int64_t K);  // below, beside the forward dispatcher

// 1: small-M input gradients run k_gemv_bwd when the caller gives a workspace.
#ifndef STM_GEMV_BWD
#define STM_GEMV_BWD 1
#endif

bool use_gemv_bwd(int64_t M, int64_t N, int64_t K, int num_groups) {
    return STM_GEMV_BWD && num_groups == 1 && M >= 1 && M <= GB_MAX_M && N > 0 && K > 0;
}

// Small-M input gradient: reduction ranges (in groups of 256 weight rows, 128
// above 16 rows) that minimise rounds x (fixed cost + groups per range) over the
// 256-column work-groups, plus STM_GEMV_BWD_PART_MB groups per MB of fp32
// partials (written by the ranges, read by the reduce); returns the range
// count and sets the groups per range. Against forced range counts over ten
// weight shapes at M = 1, 16, 32 and 64, the partials term took the picks from
// up to 8 % above the best measured count (many ranges at M = 32-64 on short
// weights, e.g. [3072,1024] M = 64 15.8 against 14.6 us) to within 4 % on all 40.
#ifndef STM_GEMV_BWD_PART_MB
#define STM_GEMV_BWD_PART_MB 0.4
#endif
int gemv_bwd_splits(int64_t M, int64_t N, int64_t K, int* groups_per_split) {
    const int64_t gn = M <= 16 ? GbCfg<1>::GN : M <= 32 ? GbCfg<2>::GN : GbCfg<4>::GN;
    const int64_t blocks = (K + GbCfg<1>::KW - 1) / GbCfg<1>::KW, groups = (N + gn - 1) / gn;
    int64_t best_gps = groups > 0 ? groups : 1;
    double best_t = 1e30;
    for (int64_t sp = 1; sp <= groups && sp <= 64; ++sp) {
        const int64_t gps = (groups + sp - 1) / sp, spe = (groups + gps - 1) / gps;
        const int64_t rounds = (blocks * spe + kCUs - 1) / kCUs;
        const double t = (double)rounds * (STM_GEMV_T_LAT + (double)gps) +
                         STM_GEMV_BWD_PART_MB * 1e-6 * (double)(spe * M * K * 4);
        if (t < best_t - 1e-9) best_t = t, best_gps = gps;
    }
    if (groups_per_split) *groups_per_split = (int)best_gps;
    return groups > 0 ? (int)((groups + best_gps - 1) / best_gps) : 1;  // every range non-empty
}

int64_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, bool backward, int num_groups) {
    // small M: room for either kernel (a pinned tile kind skips the small-M one)
    int64_t gemv_need = 0;
    if (!backward && use_gemv(M, num_groups) && !gemv_ks_tiles(M, N, K)) {
        const int sp = gemv_plan(M, N, K).splits;
        gemv_need = sp > 1 ? (int64_t)sp * M * N * (int64_t)sizeof(float) : 0;
    }
    if (backward && use_gemv_bwd(M, N, K, num_groups))  // partials even for one range (the reduce adds LoRA)
        gemv_need = (int64_t)gemv_bwd_splits(M, N, K, nullptr) * M * K * (int64_t)sizeof(float);
    const int sp = gemm_splits(M, N, K, backward, num_groups);
    const int64_t need = sp > 1 ? (int64_t)sp * M * (backward ? K : N) * (int64_t)sizeof(float) : 0;
    return need > gemv_need ? need : gemv_need;
}

#ifndef STM_FWD_R8_AUTO
#define STM_FWD_R8_AUTO 1
#endif
// Longest reduction the automatic choice runs on the 8-wave forward. Measured
// (auto plans, same box, µs, 4-wave against 8-wave): K = 4096 and 14336 at
// M = 1024-4096: 116.3 / 118.3, 224.5 / 230.6, 442.5 / 458.2 ([14336,4096]),
// 410.2 / 431.0 ([4096,14336] at M = 4096), 126.2 / 130.2 ([4096,4096]); at
// K = 1024-2048 the 8-wave kernel is 1-7 % faster (shorter per-item fixed cost).
#ifndef STM_FWD_R8_MAX_K
#define STM_FWD_R8_MAX_K 2048
#endif

// 1: small-M forwards that fit k_gemv_ks run it (no split reduction).
#ifndef STM_GEMV_KS
#define STM_GEMV_KS 1
#endif

// Configuration of the split-free small-M forward (k_gemv_ks), encoded as
// T | TW << 4 | XR << 8, or 0 when none applies: the activation rows must fit
// (M <= XR) and the launch must keep three quarters of the CUs busy, or, when
// no configuration does and the reduction is at most 16 groups (K <= 4096),
// half of them. Among the fits, the least estimated time: rounds x (fixed cost
// + tile-groups per wave), the fixed cost (level table, first copies) counted
// as one tile-group and a tile-group of a one-tile wave as 1.25 (half the work
// between barriers). At 128-191 work-groups against the split kernel
// (event-timed, µs): K <= 4096 faster, e.g. [4096,4096] M = 8 12.2 -> 10.0,
// [2048,4096] M = 1 10.8 -> 7.6, [8192,1024] M = 12 10.5 -> 7.6, [8192,4096]
// M = 16 14.3 / 14.5; K >= 11008 slower ([4096,14336] M = 8 17.5 / 20.2).
int gemv_ks_config(int64_t M, int64_t N, int64_t K) {
    if (!STM_GEMV_KS || M < 1 || M > 16) return 0;
    static const int cfgs[][3] = {{1, 1, 4}, {2, 1, 8}, {4, 1, 16}, {8, 1, 16}, {4, 2, 4}};
    const int64_t groups = (K + GV_GK - 1) / GV_GK, cus = device_cus();
    int best = 0;
    for (int pass = 0; pass < 2 && !best; ++pass) {
        if (pass == 1 && groups > 16) break;
        double best_t = 1e30;
        for (const auto& c : cfgs) {
            const int T = c[0], TW = c[1], XR = c[2], S = 8 * TW / T;
            if (M > XR) continue;
            const int64_t blocks = (N + 16 * T - 1) / (16 * T);
            if (pass == 0 ? blocks * 4 < cus * 3 : blocks * 2 < cus) continue;
            const int64_t rounds = (blocks + cus - 1) / cus;
            const double t = (double)rounds * (1.0 + (double)((groups + S - 1) / S) * TW * (TW == 1 ? 1.25 : 1.0));
            if (t < best_t) best_t = t, best = T | TW << 4 | XR << 8;
        }
    }
    return best;
}
int gemv_ks_tiles(int64_t M, int64_t N, int64_t K) { return gemv_ks_config(M, N, K); }

int launch_gemv_ks(const GemmArgs& g, int cfg, int dtype, hipStream_t stream) {
    const int T = cfg & 15;
    const dim3 grid((unsigned)((g.N + 16 * T - 1) / (16 * T))), block(512);
#define STM_KS_LAUNCH(TT, TW, XR)                                                           \
    if (dtype == STM_BF16)                                                                  \
        hipLaunchKernelGGL((k_gemv_ks<BF16, TT, TW, XR>), grid, block, 0, stream, g);       \
    else                                                                                    \
        hipLaunchKernelGGL((k_gemv_ks<F16, TT, TW, XR>), grid, block, 0, stream, g);
    switch (cfg) {
        case 1 | 1 << 4 | 4 << 8: STM_KS_LAUNCH(1, 1, 4) break;
        case 2 | 1 << 4 | 8 << 8: STM_KS_LAUNCH(2, 1, 8) break;
        case 4 | 1 << 4 | 16 << 8: STM_KS_LAUNCH(4, 1, 16) break;
        case 8 | 1 << 4 | 16 << 8: STM_KS_LAUNCH(8, 1, 16) break;
        case 4 | 2 << 4 | 4 << 8: STM_KS_LAUNCH(4, 2, 4) break;
        default: return set_error(STM_ERR_INVALID, "gemm_fwd: small-M configuration %d", cfg);
    }
#undef STM_KS_LAUNCH
    return check_launch("gemm_fwd (small M, one launch)");
}

// 1: grouped forwards whose experts hold at most 64 rows run the
// weight-streaming kernel.
#ifndef STM_GEMV_GROUPED
#define STM_GEMV_GROUPED 1
#endif

// Grouped forward with at most 64 rows per expert (the caller's max_rows, so
// decode-sized MoE batches): one work-group per (block of weight rows,
// expert), each over the whole reduction (no partials, no workspace); an
// empty expert's work-groups leave at once. The tile path would run 192- or
// 256-row tiles of MFMAs for each expert's few rows.
int launch_gemv_grouped(GemmArgs g, int dtype, hipStream_t stream) {
    g.splits = 1;
#define STM_GG_LAUNCH(MB, GKV)                                                                          \
    {                                                                                                   \
        const int ng = (int)((g.K + GKV - 1) / GKV);                                                    \
        const dim3 grid((unsigned)((g.N + GvCfg<MB, GKV>::ROWS - 1) / GvCfg<MB, GKV>::ROWS),            \
                        (unsigned)g.num_groups),                                                        \
            block(64 * GvCfg<MB, GKV>::WAVES);                                                          \
        if (dtype == STM_BF16)                                                                          \
            hipLaunchKernelGGL((k_gemv_fwd<BF16, MB, GKV, true>), grid, block, 0, stream, g, ng);      \
        else                                                                                            \
            hipLaunchKernelGGL((k_gemv_fwd<F16, MB, GKV, true>), grid, block, 0, stream, g, ng);       \
    }
    if (g.M <= 16)
        STM_GG_LAUNCH(1, 256)
    else if (g.M <= 32)
        STM_GG_LAUNCH(2, 128)
    else if (g.M <= 48)
        STM_GG_LAUNCH(3, 128)
    else if (g.M <= 64)
        STM_GG_LAUNCH(4, 128)
    else
        return set_error(STM_ERR_INVALID, "grouped gemm_fwd (small M): %lld rows per expert", (long long)g.M);
#undef STM_GG_LAUNCH
    return check_launch("grouped gemm_fwd (small M)");
}

int launch_gemm_fwd(const GemmArgs& g0, int dtype, hipStream_t stream) {
    GemmArgs g = g0;
    if (g.offsets && STM_GEMV_GROUPED && g.M >= 1 && g.M <= STM_GEMV_MAX_M && g.num_groups <= 65535 && !g.bias &&
        g.lora_rank == 0 && tile_override() < 0)
        return launch_gemv_grouped(g, dtype, stream);
    // small M: the weight-streaming kernel, when its partials have a workspace
    // (or it needs none) and the LoRA term can go to the reduce; not for a
    // grouped call (its rows come from the offsets, even with one expert)
    if (!g.offsets && use_gemv(g.M, g.num_groups) && tile_override() < 0) {
        const int kt = gemv_ks_tiles(g.M, g.N, g.K);
        if (kt) return launch_gemv_ks(g, kt, dtype, stream);
        const GemvPlan gp = gemv_plan(g.M, g.N, g.K);
        if (gp.splits == 1 ? g.lora_rank == 0 : g.partial != nullptr) return launch_gemv_fwd(g, gp, dtype, stream);
    }
    const Plan p = plan(g.M, g.N, g.K, false, g.num_groups);
    g.splits = (g.partial && p.splits > 1) ? p.splits : 1;
    const bool rw = STM_FWD_RW && rw_split_ok(false, g.splits, g.K / BK) && rw_offsets_fit(g);
    int rc;
    // unsplit single-matrix 256 x 256 tiles up to 4096 rows and reductions up to
    // STM_FWD_R8_MAX_K run the 8-wave kernel (1-7 % faster at K = 1024-2048;
    // slower at M = 8192 and on longer reductions, which keep the 4-wave
    // kernel); pinned kinds keep their kernel
    const bool auto_r8 = STM_FWD_R8_AUTO && p.kind == kBig && tile_override() < 0 && g.num_groups == 1 &&
                         g.splits == 1 && g.M <= 4096 && g.K <= STM_FWD_R8_MAX_K;
    if (p.kind == kBig && g.group_bm == 192 && g.num_groups > 1 && g.splits == 1 && rw && tile_override() < 0)
        rc = launch_fwd_rw<192, 1>(g, dtype, stream);
    else if ((p.kind == kBig8 || auto_r8) && rw_offsets_fit(g))
        rc = launch_fwd_r8(g, dtype, stream);
    else if (p.kind == kMid && rw_offsets_fit(g))
        rc = launch_fwd_rw<128, 1>(g, dtype, stream);
    else if (p.kind == kBig || p.kind == kMid || p.kind == kBig8)
        rc = rw ? launch_fwd_rw<256, STM_FWD_RW_WM>(g, dtype, stream)
                : launch_fwd_cfg<STM_FWD_BM, STM_FWD_BN, STM_FWD_WM, STM_FWD_WN>(g, dtype, stream);
    else
        rc = launch_fwd_cfg<128, 128, 2, 2>(g, dtype, stream);
    if (rc != STM_OK || g.splits == 1) return rc;
    return launch_split_reduce(g, g.N, g.bias, dtype, stream);
}

int launch_gemv_bwd(GemmArgs g, int dtype, hipStream_t stream) {
    int gps = 1;
    g.splits = gemv_bwd_splits(g.M, g.N, g.K, &gps);
    const int64_t tiles = (g.K + GbCfg<1>::KW - 1) / GbCfg<1>::KW * g.splits;  // k_gemv_bwd deals them per XCD
    const dim3 grid((unsigned)((tiles + 7) / 8 * 8)), block(512);
#define STM_GB_LAUNCH(MB)                                                              \
    if (dtype == STM_BF16)                                                             \
        hipLaunchKernelGGL((k_gemv_bwd<BF16, MB>), grid, block, 0, stream, g, gps);   \
    else                                                                               \
        hipLaunchKernelGGL((k_gemv_bwd<F16, MB>), grid, block, 0, stream, g, gps);
    if (g.M <= 16) {
        STM_GB_LAUNCH(1)
    } else if (g.M <= 32) {
        STM_GB_LAUNCH(2)
    } else {
        STM_GB_LAUNCH(4)
    }
#undef STM_GB_LAUNCH
    const int rc = check_launch("gemm_bwd_dx (small M)");
    if (rc != STM_OK) return rc;
    return launch_split_reduce(g, g.K, nullptr, dtype, stream, true);
}

int launch_gemm_bwd(const GemmArgs& g0, int dtype, hipStream_t stream) {
    // small M: the weight-streaming kernel when the caller gives a workspace for
    // its partials (sized by gemm_workspace_bytes)
    if (!g0.offsets && use_gemv_bwd(g0.M, g0.N, g0.K, g0.num_groups) && g0.partial && tile_override() < 0)
        return launch_gemv_bwd(g0, dtype, stream);
    GemmArgs g = g0;
    const Plan p = plan(g.M, g.K, g.N, true, g.num_groups);
    g.splits = (g.partial && p.splits > 1) ? p.splits : 1;
    const bool rw = STM_BWD_RW && rw_split_ok(true, g.splits, g.N / BK) && rw_offsets_fit_bwd(g);
    int rc;
    if (p.kind == kMid && rw_offsets_fit_bwd(g))
        rc = launch_bwd_rw<128>(g, dtype, stream);
    else if (p.kind == kBig || p.kind == kMid || p.kind == kBig8)
        rc = rw ? launch_bwd_rw<256>(g, dtype, stream)
                : launch_bwd_cfg<STM_BWD_BM, STM_BWD_BN, STM_BWD_WM, STM_BWD_WN>(g, dtype, stream);
    else
        rc = launch_bwd_cfg<128, 128, 2, 2>(g, dtype, stream);
    if (rc != STM_OK || g.splits == 1) return rc;
    return launch_split_reduce(g, g.K, nullptr, dtype, stream);
}

}  // namespace stm
