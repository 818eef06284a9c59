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
#define STM_GROUP_M 8
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

#ifndef STM_SWZ
#define STM_SWZ 1
#endif
__device__ __forceinline__ int swz_key(int row) { return STM_SWZ ? ((row >> 1) & 7) : (row & 7); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * 8 + (chunk ^ swz_key(row)); }

typedef __attribute__((address_space(3))) uint4 lds_uint4;

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
// one XCD reuse the same activation rows and weight rows.
__device__ __forceinline__ void tile_coords(int64_t pid, int64_t ntm, int64_t ntn, int64_t& tm, int64_t& tn) {
    const int64_t T = ntm * ntn;
    const int64_t T8 = (T / 8) * 8;
    if (pid < T8) pid = (pid % 8) * (T / 8) + pid / 8;
    const int64_t per_group = (int64_t)STM_GROUP_M * ntn;
    const int64_t grp = pid / per_group;
    const int64_t first = grp * STM_GROUP_M;
    const int64_t gsize = (ntm - first) < STM_GROUP_M ? (ntm - first) : STM_GROUP_M;
    const int64_t in = pid % per_group;
    tm = first + in % gsize;
    tn = in / gsize;
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

// Level table: entry (byte b, copy c) = (level[b >> 4], level[b & 15]) at
// index 16 b + c. Lane l reads copy l % 16, so the 16 lanes of one LDS pass of
// a 64-bit read always hit 16 different bank pairs (a single shared copy makes
// random byte values collide on banks several times per read).
constexpr int LUT_COPIES = 16;

template <int NT>
__device__ __forceinline__ void fill_lut(float2* lut, int tid) {
    for (int t = tid; t < 256 * LUT_COPIES; t += NT) {
        const int b = t / LUT_COPIES;
        lut[t] = make_float2(kLevelsDev[b >> 4], kLevelsDev[b & 15]);
    }
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
template <typename Tr, int FA, int FB>
__device__ __forceinline__ void lora_term(f32x16_t (&acc)[FA][FB], const uint16_t* __restrict__ wside,
                                          int64_t wrow_base, int64_t wrows, const uint16_t* __restrict__ xside,
                                          int64_t xrow_base, int64_t xrows, int R, int lane) {
    for (int r0 = 0; r0 < R; r0 += 16) {
        uint4 a[FA], b[FB];
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            int64_t row = wrow_base + i * 32 + (lane & 31);
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
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t col = ocol_base + i * 32 + 8 * q + 4 * (lane >> 5);
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = acc[i][j][4 * q + e];
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
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t col = ocol_base + i * 32 + 8 * q + 4 * (lane >> 5);
                if (col + 3 < ocols) {
                    *reinterpret_cast<float4*>(dst + col) =
                        make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < ocols) dst[col + e] = acc[i][j][4 * q + e];
                }
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

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    fill_lut<NT>(lut_all, tid);

    const Group grp = group_of(g, blockIdx.y);
    const int64_t K = g.K, N = g.N;
    const int64_t ntm = (g.M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
    int64_t tm, tn;
    tile_coords(blockIdx.x, ntm, ntn, tm, tn);
    const int64_t m0 = tm * BM, n0 = tn * BN;
    if (m0 >= grp.rows) return;

    int s_begin, KT;
    split_range((int)(K / BK), g.splits, blockIdx.z, s_begin, KT);
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
    if (g.lora_rank > 0 && blockIdx.z == 0)
        lora_term<Tr, FW, FX>(acc, reinterpret_cast<const uint16_t*>(g.lora_w), col_base, N,
                              reinterpret_cast<const uint16_t*>(g.lora_x) + grp.row0 * g.lora_rank, row_base,
                              grp.rows, g.lora_rank, lane);
    if (g.splits > 1)
        store_tile_f32<FW, FX>(acc, g.partial + (int64_t)blockIdx.z * g.M * N, N, col_base, N, row_base, grp.rows,
                               lane);
    else
        store_tile<Tr, FW, FX>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * N, N, col_base, N, row_base,
                               grp.rows, reinterpret_cast<const uint16_t*>(g.bias), lane);
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

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    fill_lut<NT>(lut_all, tid);

    const Group grp = group_of(g, blockIdx.y);
    const int64_t K = g.K, N = g.N;
    const int64_t ntm = (g.M + BM - 1) / BM, ntk = (K + BN - 1) / BN;
    int64_t tm, tk;
    tile_coords(blockIdx.x, ntm, ntk, tm, tk);
    const int64_t m0 = tm * BM, k0 = tk * BN;
    if (m0 >= grp.rows) return;

    int s_begin, NT_steps;
    split_range((int)(N / BK), g.splits, blockIdx.z, s_begin, NT_steps);
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
    if (g.lora_rank > 0 && blockIdx.z == 0)
        lora_term<Tr, FW, FX>(acc, reinterpret_cast<const uint16_t*>(g.lora_w), col_base, K,
                              reinterpret_cast<const uint16_t*>(g.lora_x) + grp.row0 * g.lora_rank, row_base,
                              grp.rows, g.lora_rank, lane);
    if (g.splits > 1)
        store_tile_f32<FW, FX>(acc, g.partial + (int64_t)blockIdx.z * g.M * K, K, col_base, K, row_base, grp.rows,
                               lane);
    else
        store_tile<Tr, FW, FX>(acc, reinterpret_cast<uint16_t*>(g.out) + grp.row0 * K, K, col_base, K, row_base,
                               grp.rows, nullptr, lane);
}

// Sum of the split partials [splits][rows][cols] (+ bias), one rounding; four
// columns per lane (cols % 4 == 0).
template <typename Tr>
__global__ __launch_bounds__(256) void k_split_reduce(const float* __restrict__ partial, int splits, int64_t rows,
                                                      int64_t cols, const uint16_t* __restrict__ bias,
                                                      uint16_t* __restrict__ out) {
    const int64_t total = rows * (cols / 4), plane = rows * cols;
    for (int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; v < total; v += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = v * 4;
        float4 acc = *reinterpret_cast<const float4*>(partial + e);
        for (int z = 1; z < splits; ++z) {
            const float4 p = *reinterpret_cast<const float4*>(partial + z * plane + e);
            acc.x += p.x;
            acc.y += p.y;
            acc.z += p.z;
            acc.w += p.w;
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

int launch_split_reduce(const GemmArgs& g, int64_t cols, const void* bias, int dtype, hipStream_t stream) {
    const int64_t items = g.M * (cols / 4);
    if (items == 0) return STM_OK;
    const int64_t blocks = (items + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 16384 ? blocks : 16384);
    if (dtype == STM_BF16)
        hipLaunchKernelGGL(k_split_reduce<BF16>, dim3(grid), dim3(256), 0, stream, g.partial, g.splits, g.M, cols,
                           (const uint16_t*)bias, (uint16_t*)g.out);
    else
        hipLaunchKernelGGL(k_split_reduce<F16>, dim3(grid), dim3(256), 0, stream, g.partial, g.splits, g.M, cols,
                           (const uint16_t*)bias, (uint16_t*)g.out);
    return check_launch("gemm split reduce");
}

template <int BM, int BN, int WM, int WN>
int launch_fwd_cfg(const GemmArgs& g, int dtype, hipStream_t stream) {
    const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    if (tiles == 0) return STM_OK;
    if (tiles > 0x7FFFFFFFLL || g.num_groups > 65535) return set_error(STM_ERR_UNSUPPORTED, "gemm_fwd: grid too large");
    dim3 grid((unsigned)tiles, (unsigned)g.num_groups, (unsigned)g.splits), block(WM * WN * 64);
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
    if (tiles > 0x7FFFFFFFLL || g.num_groups > 65535)
        return set_error(STM_ERR_UNSUPPORTED, "gemm_bwd_dx: grid too large");
    dim3 grid((unsigned)tiles, (unsigned)g.num_groups, (unsigned)g.splits), block(WM * WN * 64);
    if (dtype == STM_BF16)
        hipLaunchKernelGGL((k_gemm_bwd<BF16, BM, BN, WM, WN>), grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL((k_gemm_bwd<F16, BM, BN, WM, WN>), grid, block, 0, stream, g);
    return check_launch("gemm_bwd_dx");
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
// big tile, 0.8 us 128 x 128; input gradient: 2.4 us, 1.35 us), t_wave = 8 us
// of per-tile prologue and epilogue, reduce = the fp32 partials written and
// read once at 5 TB/s plus 4 us. Splits: at most 16, at least 8 steps each;
// grouped launches never split.
constexpr int kCUs = 256;

struct Plan {
    bool big;
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

Plan plan(int64_t M, int64_t cols, int64_t red, bool backward, int num_groups) {
    const int64_t bm = backward ? STM_BWD_BM : STM_FWD_BM, bn = backward ? STM_BWD_BN : STM_FWD_BN;
    const int64_t big_tiles = ((M + bm - 1) / bm) * ((cols + bn - 1) / bn) * num_groups;
    const int64_t small_tiles = ((M + 127) / 128) * ((cols + 127) / 128) * num_groups;
    const int64_t steps = red / BK;
    const double t_big = backward ? 2.4 : 2.0, t_small = backward ? 1.35 : 0.8;
    int max_sp = 1;
    if (num_groups == 1) {
        const int64_t by_steps = steps / 8;
        max_sp = (int)(by_steps < 16 ? (by_steps > 1 ? by_steps : 1) : 16);
    }
    Plan best{true, big_tiles, 1};
    double best_t = plan_cost(big_tiles, steps, 1, t_big, M, cols);
    for (int sp = 1; sp <= max_sp; ++sp) {
        const double tb = plan_cost(big_tiles, steps, sp, t_big, M, cols);
        if (tb < best_t) {
            best_t = tb;
            best = Plan{true, big_tiles, sp};
        }
        const double ts = plan_cost(small_tiles, steps, sp, t_small, M, cols);
        if (ts < best_t) {
            best_t = ts;
            best = Plan{false, small_tiles, sp};
        }
    }
    return best;
}

}  // namespace

int gemm_splits(int64_t M, int64_t N, int64_t K, bool backward, int num_groups) {
    return backward ? plan(M, K, N, true, num_groups).splits : plan(M, N, K, false, num_groups).splits;
}

int64_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, bool backward, int num_groups) {
    const int sp = gemm_splits(M, N, K, backward, num_groups);
    return sp > 1 ? (int64_t)sp * M * (backward ? K : N) * (int64_t)sizeof(float) : 0;
}

int launch_gemm_fwd(const GemmArgs& g0, int dtype, hipStream_t stream) {
    GemmArgs g = g0;
    const Plan p = plan(g.M, g.N, g.K, false, g.num_groups);
    g.splits = (g.partial && p.splits > 1) ? p.splits : 1;
    const int rc = p.big ? launch_fwd_cfg<STM_FWD_BM, STM_FWD_BN, STM_FWD_WM, STM_FWD_WN>(g, dtype, stream)
                         : launch_fwd_cfg<128, 128, 2, 2>(g, dtype, stream);
    if (rc != STM_OK || g.splits == 1) return rc;
    return launch_split_reduce(g, g.N, g.bias, dtype, stream);
}

int launch_gemm_bwd(const GemmArgs& g0, int dtype, hipStream_t stream) {
    GemmArgs g = g0;
    const Plan p = plan(g.M, g.K, g.N, true, g.num_groups);
    g.splits = (g.partial && p.splits > 1) ? p.splits : 1;
    const int rc = p.big ? launch_bwd_cfg<STM_BWD_BM, STM_BWD_BN, STM_BWD_WM, STM_BWD_WN>(g, dtype, stream)
                         : launch_bwd_cfg<128, 128, 2, 2>(g, dtype, stream);
    if (rc != STM_OK || g.splits == 1) return rc;
    return launch_split_reduce(g, g.K, nullptr, dtype, stream);
}

}  // namespace stm
