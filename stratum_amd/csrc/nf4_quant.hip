// NF4 blockwise quantize + nibble pack, and dequantize, for gfx950.
//
// quantize: one lane owns 8 consecutive elements (one 16-byte load of fp16/bf16),
//   the L = blocksize/8 lanes of a block reduce max|x| with cross-lane shuffles,
//   every element picks its level from a 65-cell table held in LDS, and each
//   lane stores its 8 codes as one 32-bit word, so a wave writes 256 contiguous
//   bytes of packed codes per iteration.
// dequantize: one lane owns one 32-bit word of packed codes (8 elements), looks
//   each byte up in a 256-entry (level_hi, level_lo) table in LDS, multiplies by
//   the block's absmax in fp32 and stores 16 bytes of fp16/bf16 (32 of fp32).
#include <type_traits>

#include "nf4_kernels.h"

namespace stm {

#pragma clang fp contract(off)

// Tensors per batched (de)quantize launch; their pointers and sizes travel as
// kernel arguments (under 2 KB).
constexpr int kManyMax = 32;

template <int DT>
using Tr16 = std::conditional_t<DT == STM_BF16, BF16, F16>;

// max that propagates NaN (IEEE 754-2019 maximum: v_maximum3_f32 on gfx950,
// which also takes |x| as a free source modifier) -- a block holding a NaN has
// a NaN absmax, as torch.max gives the reference.
__device__ __forceinline__ float nanmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Level of s = x / absmax. s is clamped to [-1, 1] (v_med3_f32: +-inf from an
// absmax whose reciprocal overflows go to +-1, as the CPU rule's clamp does).
// The cell index comes from the bits of f = c * 32 + (2^21 + 32) (one
// rounding; c * 32 is exact): in [2^21, 2^22) the float spacing is 1/4, so the
// low mantissa bits of f hold round(128 c + 128) in [0, 256], and those bits &
// 0x3FC are 4 * cell (cell in [0, 64]) -- already the byte offset of the
// cell's entry, with no convert or shift. A NaN s (all-zero or NaN block)
// gives f = NaN whose bits & 0x3FC are 0, and c = -1 gives f = 2^21, also
// cell 0, whose base is code 0 and whose bound (2.0) is never met -- code 0,
// as both bitsandbytes rules give. v_med3_f32 with a NaN operand returns the
// minimum of its operands (IEEE mode: the smaller non-NaN one), so a NaN s of
// any payload becomes c = -1; should a NaN c still reach the formula, its
// payload bits can name any cell up to 255, and the LDS tables are padded to
// 256 cells with copies of cell 0 (see fill_cells), so the read stays inside
// the tables and the code is still 0 for the cells above 64.
__device__ __forceinline__ uint32_t level_of(float s, const float* __restrict__ bound,
                                             const uint32_t* __restrict__ base) {
    const float c = __builtin_amdgcn_fmed3f(s, -1.0f, 1.0f);
    const uint32_t j = (__float_as_uint(__builtin_fmaf(c, 32.0f, 2097184.0f)) & 0x3FCu) >> 2;
    return base[j] + (c >= bound[j] ? 1u : 0u);
}

// LDS copies of the cell table: cells 0..64 from the host table, 65..255 as
// cell 0 (bound 2.0 is never met, base code 0), one cell per thread.
constexpr int kLdsCells = 256;
__device__ __forceinline__ void fill_cells(const CellTable& tab, float* s_bound, uint32_t* s_base, int tid,
                                           int nthreads) {
    for (int t = tid; t < kLdsCells; t += nthreads) {
        s_bound[t] = t < 65 ? tab.bound[t] : 2.0f;
        s_base[t] = t < 65 ? tab.base[t] : 0u;
    }
}

template <int DT>
__device__ __forceinline__ float load1(const void* x, int64_t i) {
    if constexpr (DT == STM_F32)
        return reinterpret_cast<const float*>(x)[i];
    else
        return Tr16<DT>::to_f32(reinterpret_cast<const uint16_t*>(x)[i]);
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// fp32(half h of w) * r, one rounding: v_fma_mix_f32 with a zero addend (the
// conversion of the fp16 operand is exact), one VALU op for convert + scale.
template <int HI>
__device__ __forceinline__ float f16_times(uint32_t w, float r) {
    float s;
    if constexpr (HI)
        __asm__("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(s) : "v"(w), "v"(r));
    else
        __asm__("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(s) : "v"(w), "v"(r));
    return s;
}
// per-half IEEE maximum of three packed fp16 pairs (NaN-propagating)
__device__ __forceinline__ uint32_t pk_max3_f16(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t d;
    __asm__("v_pk_maximum3_f16 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}
#pragma clang diagnostic pop

// One lane's 8 elements of a chunk: 16-bit inputs stay packed (4 words),
// fp32 inputs are 8 floats.
template <int DT>
struct Chunk8 {
    uint4 w;
    __device__ __forceinline__ void load(const void* __restrict__ x, int64_t g) {
        w = reinterpret_cast<const uint4*>(x)[g];
    }
    __device__ __forceinline__ void zero() { w = make_uint4(0u, 0u, 0u, 0u); }
    __device__ __forceinline__ uint32_t word(int k) const { return k == 0 ? w.x : k == 1 ? w.y : k == 2 ? w.z : w.w; }
    // element 2k + h scaled by r, in fp32 (one rounding)
    __device__ __forceinline__ float scaled(int k, int h, float r) const {
        if constexpr (DT == STM_F16)
            return h ? f16_times<1>(word(k), r) : f16_times<0>(word(k), r);
        else
            return (h ? __uint_as_float(word(k) & 0xFFFF0000u) : __uint_as_float(word(k) << 16)) * r;
    }
};
template <>
struct Chunk8<STM_F32> {
    float v[8];
    __device__ __forceinline__ void load(const void* __restrict__ x, int64_t g) {
        const float4* p = reinterpret_cast<const float4*>(x) + 2 * g;
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    }
    __device__ __forceinline__ float scaled(int k, int h, float r) const { return v[2 * k + h] * r; }
};

// max|x| over a lane's C chunks, in fp32 (NaN-propagating). fp16: per-half
// maxima of |x| on the packed words (v_pk_maximum3_f16 on x & 0x7FFF7FFF),
// then the two halves, then one exact conversion; the others in fp32.
template <int DT, int C>
__device__ __forceinline__ float lane_absmax(const Chunk8<DT> (&ch)[C]) {
    if constexpr (DT == STM_F16) {
        uint32_t m = ch[0].w.x & 0x7FFF7FFFu;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const uint32_t a = ch[c].w.x & 0x7FFF7FFFu, b = ch[c].w.y & 0x7FFF7FFFu;
            const uint32_t d = ch[c].w.z & 0x7FFF7FFFu, e = ch[c].w.w & 0x7FFF7FFFu;
            m = pk_max3_f16(pk_max3_f16(m, a, b), d, e);
        }
        m = pk_max3_f16(m, m >> 16, m);  // low half: max of both halves (the high half of m >> 16 is +0)
        return (float)__builtin_bit_cast(_Float16, (uint16_t)(m & 0xFFFFu));
    } else if constexpr (DT == STM_BF16) {
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                a = nanmax(nanmax(a, fabsf(__uint_as_float(ch[c].word(k) << 16))),
                           fabsf(__uint_as_float(ch[c].word(k) & 0xFFFF0000u)));
        return a;
    } else {
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int e = 0; e < 8; ++e) a = nanmax(a, fabsf(ch[c].v[e]));
        return a;
    }
}

// L lanes per quantization block, C 8-element chunks per lane: blocksize = 8 * L * C.
// A wave handles U rounds of 64 / L consecutive blocks. All its loads are
// issued first (U * C 16-byte loads per lane in flight), then the cell table
// is copied to LDS -- so the table setup and the barrier overlap the HBM
// latency. The U rounds' absmax values are reduced first; lane u of each
// block's L lanes then computes the reciprocal for round u (one IEEE division
// per lane instead of U), which the group's lanes read back with a shuffle.
// Then each round is quantized and stored. Every thread reaches the barrier;
// rounds past the end are masked.
template <int DT, int L, int C, int U>
__device__ __forceinline__ void quantize_workgroup(const void* __restrict__ x, uint32_t* __restrict__ packed,
                                                   float* __restrict__ absmax, int64_t nblocks, int64_t wg,
                                                   const CellTable& tab, float* s_bound, uint32_t* s_base) {
    static_assert(U <= L, "one reciprocal per lane of a block's group");
    constexpr int BPW = 64 / L;  // blocks per round
    constexpr int GPB = L * C;   // 8-element groups per block
    const int lane = threadIdx.x & 63;
    const int64_t wave = (wg * 256 + threadIdx.x) >> 6;
    const int64_t first = wave * (BPW * U);

    Chunk8<DT> ch[U][C];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t blk = first + u * BPW + lane / L;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            if (blk < nblocks)
                ch[u][c].load(x, blk * GPB + c * L + (lane % L));
            else
                ch[u][c].zero();
        }
    }
    fill_cells(tab, s_bound, s_base, threadIdx.x, 256);
    __syncthreads();

    float a[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        a[u] = lane_absmax<DT, C>(ch[u]);
#pragma unroll
        for (int off = 1; off < L; off <<= 1) a[u] = nanmax(a[u], __shfl_xor(a[u], off));
    }
    float r[U];
    if constexpr (U == 1) {
        r[0] = 1.0f / a[0];  // IEEE division (correctly rounded)
    } else {
        const int k = lane % L;
        float mine = a[0];
#pragma unroll
        for (int u = 1; u < U; ++u) mine = k == u ? a[u] : mine;
        const float inv = 1.0f / mine;  // IEEE division (correctly rounded), round k's for lanes k < U
        const int group = lane & ~(L - 1);
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = __shfl(inv, group + u);
    }

#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t blk = first + u * BPW + lane / L;
        const bool active = blk < nblocks;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            uint32_t word = 0;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t q0 = level_of(ch[u][c].scaled(p, 0, r[u]), s_bound, s_base);
                const uint32_t q1 = level_of(ch[u][c].scaled(p, 1, r[u]), s_bound, s_base);
                word |= ((q0 << 4) | q1) << (8 * p);
            }
            if (active) packed[blk * GPB + c * L + (lane % L)] = word;
        }
        if (active && (lane % L) == 0) absmax[blk] = a[u];
    }
}

template <int DT, int L, int C, int U>
__global__ __launch_bounds__(256) void k_quantize(const void* __restrict__ x, uint32_t* __restrict__ packed,
                                                  float* __restrict__ absmax, int64_t nblocks, CellTable tab) {
    __shared__ float s_bound[kLdsCells];
    __shared__ uint32_t s_base[kLdsCells];
    quantize_workgroup<DT, L, C, U>(x, packed, absmax, nblocks, blockIdx.x, tab, s_bound, s_base);
}

// Several tensors in one launch (the same dtype, blocksize and rule): tensor t
// owns work-groups [first_wg[t], first_wg[t + 1]); each work-group finds its
// tensor with a uniform scan of the (kernel-argument) prefix array.
struct QuantMany {
    CellTable tab;
    int count;
    int64_t first_wg[kManyMax + 1];
    const void* x[kManyMax];
    uint32_t* packed[kManyMax];
    float* absmax[kManyMax];
    int64_t nblocks[kManyMax];
};

__device__ __forceinline__ int tensor_of(const int64_t* first_wg, int count, int64_t wg) {
    int t = 0;
    for (int i = 1; i < count; ++i) t += wg >= first_wg[i] ? 1 : 0;
    return t;
}

template <int DT, int L, int C, int U>
__global__ __launch_bounds__(256) void k_quantize_many(QuantMany m) {
    __shared__ float s_bound[kLdsCells];
    __shared__ uint32_t s_base[kLdsCells];
    const int t = tensor_of(m.first_wg, m.count, blockIdx.x);
    quantize_workgroup<DT, L, C, U>(m.x[t], m.packed[t], m.absmax[t], m.nblocks[t], blockIdx.x - m.first_wg[t], m.tab,
                                    s_bound, s_base);
}

// One thread per block; used for a partial last block and for unaligned inputs.
template <int DT>
__global__ __launch_bounds__(64) void k_quantize_generic(const void* __restrict__ x, int64_t n, int bs,
                                                         int64_t b_begin, int64_t b_end, uint8_t* __restrict__ packed,
                                                         float* __restrict__ absmax, CellTable tab) {
    __shared__ float s_bound[kLdsCells];
    __shared__ uint32_t s_base[kLdsCells];
    fill_cells(tab, s_bound, s_base, threadIdx.x, 64);
    __syncthreads();
    const int64_t blk = b_begin + (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (blk >= b_end) return;
    const int64_t lo = blk * bs, hi = (lo + bs < n) ? lo + bs : n;
    float a = 0.0f;
    for (int64_t i = lo; i < hi; ++i) a = nanmax(a, fabsf(load1<DT>(x, i)));
    absmax[blk] = a;
    const float r = 1.0f / a;
    for (int64_t i = lo; i < hi; i += 2) {
        uint32_t q0 = level_of(load1<DT>(x, i) * r, s_bound, s_base);
        uint32_t q1 = (i + 1 < hi) ? level_of(load1<DT>(x, i + 1) * r, s_bound, s_base) : 0u;
        packed[i >> 1] = (uint8_t)((q0 << 4) | q1);
    }
}

template <int DT, int L, int C, int U>
static void quantize_launch(const void* A, int64_t nfull, const CellTable& tab, uint32_t* p4, float* absmax,
                            hipStream_t stream) {
    const int64_t per_wave = (64 / L) * U;
    const int64_t waves = (nfull + per_wave - 1) / per_wave;
    const int64_t grid = (waves + 3) / 4;
    hipLaunchKernelGGL((k_quantize<DT, L, C, U>), dim3((unsigned)grid), dim3(256), 0, stream, A, p4, absmax, nfull,
                       tab);
}

template <int DT, int L, int C, int U>
static int64_t quantize_workgroups(int64_t nfull) {
    const int64_t per_wave = (64 / L) * U;
    return ((nfull + per_wave - 1) / per_wave + 3) / 4;
}

template <int DT, int L, int C, int U>
static int quantize_many_launch(QuantMany& m, hipStream_t stream) {
    m.first_wg[0] = 0;
    for (int t = 0; t < m.count; ++t) m.first_wg[t + 1] = m.first_wg[t] + quantize_workgroups<DT, L, C, U>(m.nblocks[t]);
    if (m.first_wg[m.count] > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "quantize_many: batch too large");
    if (m.first_wg[m.count] > 0)
        hipLaunchKernelGGL((k_quantize_many<DT, L, C, U>), dim3((unsigned)m.first_wg[m.count]), dim3(256), 0, stream,
                           m);
    return STM_OK;
}

template <int DT>
static int quantize_many_dispatch(QuantMany& m, int bs, hipStream_t stream) {
    switch (bs) {
        case 64: return quantize_many_launch<DT, 8, 1, 4>(m, stream);
        case 128: return quantize_many_launch<DT, 16, 1, 4>(m, stream);
        case 256: return quantize_many_launch<DT, 32, 1, 4>(m, stream);
        case 512: return quantize_many_launch<DT, 64, 1, 4>(m, stream);
        case 1024: return quantize_many_launch<DT, 64, 2, 2>(m, stream);
        case 2048: return quantize_many_launch<DT, 64, 4, 1>(m, stream);
        default: return quantize_many_launch<DT, 64, 8, 1>(m, stream);
    }
}

template <int DT>
static int quantize_vec_dispatch(const void* A, int64_t nfull, int bs, const CellTable& tab, uint8_t* packed,
                                 float* absmax, hipStream_t stream) {
    // one work-group = 4 waves; a wave covers U * 64 / L blocks
    if ((nfull + 3) / 4 > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "quantize: n too large");
    uint32_t* p4 = reinterpret_cast<uint32_t*>(packed);
    switch (bs) {
        // rounds per wave by size (HIP-graph device time, fp16 in): a [5632, 2048]
        // weight (180 K blocks) 6.8 us with 1 against 7.6 with 4; a [14336, 4096]
        // weight (917 K blocks) keeps 4 (1: +5 %)
        case 64:
            if (nfull < ((int64_t)1 << 19))
                quantize_launch<DT, 8, 1, 1>(A, nfull, tab, p4, absmax, stream);
            else
                quantize_launch<DT, 8, 1, 4>(A, nfull, tab, p4, absmax, stream);
            break;
        case 128: quantize_launch<DT, 16, 1, 4>(A, nfull, tab, p4, absmax, stream); break;
        case 256: quantize_launch<DT, 32, 1, 4>(A, nfull, tab, p4, absmax, stream); break;
        case 512: quantize_launch<DT, 64, 1, 4>(A, nfull, tab, p4, absmax, stream); break;
        case 1024: quantize_launch<DT, 64, 2, 2>(A, nfull, tab, p4, absmax, stream); break;
        case 2048: quantize_launch<DT, 64, 4, 1>(A, nfull, tab, p4, absmax, stream); break;
        default: quantize_launch<DT, 64, 8, 1>(A, nfull, tab, p4, absmax, stream); break;
    }
    return STM_OK;
}

int launch_quantize(const void* A, int dtype, int64_t n, int bs, const CellTable& tab, uint8_t* packed,
                    float* absmax, hipStream_t stream) {
    const int64_t nblocks = (n + bs - 1) / bs;
    const bool vec_ok = aligned(A, 16) && aligned(packed, 4);
    const int64_t nfull = vec_ok ? n / bs : 0;
    if (nfull > 0) {
        int rc;
        if (dtype == STM_F16)
            rc = quantize_vec_dispatch<STM_F16>(A, nfull, bs, tab, packed, absmax, stream);
        else if (dtype == STM_BF16)
            rc = quantize_vec_dispatch<STM_BF16>(A, nfull, bs, tab, packed, absmax, stream);
        else
            rc = quantize_vec_dispatch<STM_F32>(A, nfull, bs, tab, packed, absmax, stream);
        if (rc == STM_OK) rc = check_launch("quantize");
        if (rc) return rc;
    }
    if (nfull < nblocks) {
        dim3 g((unsigned)((nblocks - nfull + 63) / 64)), b(64);
        if (dtype == STM_F16)
            hipLaunchKernelGGL(k_quantize_generic<STM_F16>, g, b, 0, stream, A, n, bs, nfull, nblocks, packed, absmax, tab);
        else if (dtype == STM_BF16)
            hipLaunchKernelGGL(k_quantize_generic<STM_BF16>, g, b, 0, stream, A, n, bs, nfull, nblocks, packed, absmax, tab);
        else
            hipLaunchKernelGGL(k_quantize_generic<STM_F32>, g, b, 0, stream, A, n, bs, nfull, nblocks, packed, absmax, tab);
        return check_launch("quantize(tail)");
    }
    return STM_OK;
}

int launch_quantize_many(int count, const void* const* A, const int64_t* n, int dtype, int bs, const CellTable& tab,
                         uint8_t* const* packed, float* const* absmax, hipStream_t stream) {
    // the whole blocks of 16-byte aligned inputs go through batched launches of
    // up to kManyMax tensors; partial last blocks and unaligned inputs take
    // the single-tensor path (its tail kernel)
    QuantMany m{};
    m.tab = tab;
    auto flush = [&]() -> int {
        if (m.count == 0) return STM_OK;
        int rc;
        if (dtype == STM_F16)
            rc = quantize_many_dispatch<STM_F16>(m, bs, stream);
        else if (dtype == STM_BF16)
            rc = quantize_many_dispatch<STM_BF16>(m, bs, stream);
        else
            rc = quantize_many_dispatch<STM_F32>(m, bs, stream);
        m.count = 0;
        return rc ? rc : check_launch("quantize_many");
    };
    for (int t = 0; t < count; ++t) {
        const int64_t nfull = (aligned(A[t], 16) && aligned(packed[t], 4)) ? n[t] / bs : 0;
        if (nfull > 0) {
            m.x[m.count] = A[t];
            m.packed[m.count] = reinterpret_cast<uint32_t*>(packed[t]);
            m.absmax[m.count] = absmax[t];
            m.nblocks[m.count] = nfull;
            if (++m.count == kManyMax) {
                const int rc = flush();
                if (rc) return rc;
            }
        }
    }
    int rc = flush();
    if (rc) return rc;
    for (int t = 0; t < count; ++t) {
        const int64_t nfull = (aligned(A[t], 16) && aligned(packed[t], 4)) ? n[t] / bs : 0;
        const int64_t nblocks = (n[t] + bs - 1) / bs;
        if (nfull == nblocks) continue;
        if (nfull == 0) {
            rc = launch_quantize(A[t], dtype, n[t], bs, tab, packed[t], absmax[t], stream);
        } else {
            dim3 g((unsigned)((nblocks - nfull + 63) / 64)), b(64);
            if (dtype == STM_F16)
                hipLaunchKernelGGL(k_quantize_generic<STM_F16>, g, b, 0, stream, A[t], n[t], bs, nfull, nblocks,
                                   packed[t], absmax[t], tab);
            else if (dtype == STM_BF16)
                hipLaunchKernelGGL(k_quantize_generic<STM_BF16>, g, b, 0, stream, A[t], n[t], bs, nfull, nblocks,
                                   packed[t], absmax[t], tab);
            else
                hipLaunchKernelGGL(k_quantize_generic<STM_F32>, g, b, 0, stream, A[t], n[t], bs, nfull, nblocks,
                                   packed[t], absmax[t], tab);
            rc = check_launch("quantize_many(tail)");
        }
        if (rc) return rc;
    }
    return STM_OK;
}

// ------------------------------------------------------------------ dequant
template <int DT>
__device__ __forceinline__ void store8(void* __restrict__ out, int64_t g, const float* v) {
    if constexpr (DT == STM_F32) {
        float4* o = reinterpret_cast<float4*>(out) + 2 * g;
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        uint4 r;
        r.x = Tr16<DT>::pack2(v[0], v[1]);
        r.y = Tr16<DT>::pack2(v[2], v[3]);
        r.z = Tr16<DT>::pack2(v[4], v[5]);
        r.w = Tr16<DT>::pack2(v[6], v[7]);
        reinterpret_cast<uint4*>(out)[g] = r;
    }
}

// U words of packed codes per lane, wave-contiguous: word g = (wg*U + j)*256 + tid.
template <int DT, int U>
__device__ __forceinline__ void dequantize_workgroup(const uint32_t* __restrict__ q, const float* __restrict__ absmax,
                                                     void* __restrict__ out, int64_t ngroups, int gshift, int64_t wg,
                                                     float2* lut) {
    lut[threadIdx.x] = make_float2(kLevelsDev[threadIdx.x >> 4], kLevelsDev[threadIdx.x & 15]);
    __syncthreads();
    const int64_t base = wg * (U * 256) + threadIdx.x;
    uint32_t w[U];
    float a[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int64_t g = base + j * 256;
        w[j] = 0u;
        a[j] = 0.0f;
        if (g < ngroups) {
            w[j] = q[g];
            a[j] = absmax[g >> gshift];
        }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int64_t g = base + j * 256;
        if (g < ngroups) {
            float v[8];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float2 c = lut[(w[j] >> (8 * b)) & 0xFFu];
                v[2 * b] = opaque(c.x * a[j]);
                v[2 * b + 1] = opaque(c.y * a[j]);
            }
            store8<DT>(out, g, v);
        }
    }
}

template <int DT, int U>
__global__ __launch_bounds__(256) void k_dequantize(const uint32_t* __restrict__ q, const float* __restrict__ absmax,
                                                    void* __restrict__ out, int64_t ngroups, int gshift) {
    __shared__ float2 lut[256];
    dequantize_workgroup<DT, U>(q, absmax, out, ngroups, gshift, blockIdx.x, lut);
}

// Several tensors in one launch (the same blocksize and output dtype), as QuantMany.
struct DequantMany {
    int count;
    int gshift;
    int64_t first_wg[kManyMax + 1];
    const uint32_t* q[kManyMax];
    const float* absmax[kManyMax];
    void* out[kManyMax];
    int64_t ngroups[kManyMax];
};

template <int DT, int U>
__global__ __launch_bounds__(256) void k_dequantize_many(DequantMany m) {
    __shared__ float2 lut[256];
    const int t = tensor_of(m.first_wg, m.count, blockIdx.x);
    dequantize_workgroup<DT, U>(m.q[t], m.absmax[t], m.out[t], m.ngroups[t], m.gshift, blockIdx.x - m.first_wg[t],
                                lut);
}

template <int DT>
__global__ __launch_bounds__(256) void k_dequantize_generic(const uint8_t* __restrict__ q,
                                                            const float* __restrict__ absmax, void* __restrict__ out,
                                                            int64_t start, int64_t n, int bshift) {
    const int64_t i = start + (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const uint32_t byte = q[i >> 1];
    const uint32_t code = (i & 1) ? (byte & 15u) : (byte >> 4);
    const float v = opaque(kLevelsDev[code] * absmax[i >> bshift]);
    if constexpr (DT == STM_F32)
        reinterpret_cast<float*>(out)[i] = v;
    else
        reinterpret_cast<uint16_t*>(out)[i] = Tr16<DT>::from_f32(v);
}

template <int DT, int U>
static void dequant_launch(const uint8_t* packed, const float* absmax, int64_t ngroups, int bshift, void* out,
                           hipStream_t stream) {
    dim3 g((unsigned)((ngroups + U * 256 - 1) / (U * 256))), b(256);
    hipLaunchKernelGGL((k_dequantize<DT, U>), g, b, 0, stream, reinterpret_cast<const uint32_t*>(packed), absmax, out,
                       ngroups, bshift - 3);
}

// Groups per thread by size (HIP-graph device time on MI355X, fp16 out): a
// [5632, 2048] weight (1.4 M groups) 6.1 us with 2 against 6.5 with 4; a
// [14336, 4096] weight (7.3 M groups) 23.0 us with 8 against 23.7 with 4.
template <int DT>
static void dequant_dispatch(const uint8_t* packed, const float* absmax, int64_t n, int bshift, void* out,
                             bool vec_ok, hipStream_t stream) {
    const int64_t ngroups = vec_ok ? n / 8 : 0;
    if (ngroups >= (int64_t)1 << 22)
        dequant_launch<DT, 8>(packed, absmax, ngroups, bshift, out, stream);
    else if (ngroups >= (int64_t)1 << 21)
        dequant_launch<DT, 4>(packed, absmax, ngroups, bshift, out, stream);
    else if (ngroups > 0)
        dequant_launch<DT, 2>(packed, absmax, ngroups, bshift, out, stream);
    const int64_t start = ngroups * 8;
    if (start < n) {
        dim3 g((unsigned)((n - start + 255) / 256)), b(256);
        hipLaunchKernelGGL(k_dequantize_generic<DT>, g, b, 0, stream, packed, absmax, out, start, n, bshift);
    }
}

int launch_dequantize(const uint8_t* packed, const float* absmax, int64_t n, int bs, void* out, int out_dtype,
                      hipStream_t stream) {
    const int bshift = ilog2(bs);
    const bool vec_ok = aligned(packed, 4) && aligned(out, 16);
    if ((n + 255) / 256 > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "dequantize: n too large");
    if (out_dtype == STM_F16)
        dequant_dispatch<STM_F16>(packed, absmax, n, bshift, out, vec_ok, stream);
    else if (out_dtype == STM_BF16)
        dequant_dispatch<STM_BF16>(packed, absmax, n, bshift, out, vec_ok, stream);
    else
        dequant_dispatch<STM_F32>(packed, absmax, n, bshift, out, vec_ok, stream);
    return check_launch("dequantize");
}

template <int DT>
static int dequant_many_launch(DequantMany& m, hipStream_t stream) {
    constexpr int U = 4;
    m.first_wg[0] = 0;
    for (int t = 0; t < m.count; ++t) m.first_wg[t + 1] = m.first_wg[t] + (m.ngroups[t] + U * 256 - 1) / (U * 256);
    if (m.first_wg[m.count] > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "dequantize_many: batch too large");
    if (m.first_wg[m.count] > 0)
        hipLaunchKernelGGL((k_dequantize_many<DT, U>), dim3((unsigned)m.first_wg[m.count]), dim3(256), 0, stream, m);
    return STM_OK;
}

int launch_dequantize_many(int count, const uint8_t* const* packed, const float* const* absmax, const int64_t* n,
                           int bs, void* const* out, int out_dtype, hipStream_t stream) {
    // whole 8-element groups of aligned tensors batched, the rest per tensor
    const int bshift = ilog2(bs);
    DequantMany m{};
    m.gshift = bshift - 3;
    auto flush = [&]() -> int {
        if (m.count == 0) return STM_OK;
        int rc;
        if (out_dtype == STM_F16)
            rc = dequant_many_launch<STM_F16>(m, stream);
        else if (out_dtype == STM_BF16)
            rc = dequant_many_launch<STM_BF16>(m, stream);
        else
            rc = dequant_many_launch<STM_F32>(m, stream);
        m.count = 0;
        return rc ? rc : check_launch("dequantize_many");
    };
    for (int t = 0; t < count; ++t) {
        if (!(aligned(packed[t], 4) && aligned(out[t], 16)) || n[t] < 8) continue;
        m.q[m.count] = reinterpret_cast<const uint32_t*>(packed[t]);
        m.absmax[m.count] = absmax[t];
        m.out[m.count] = out[t];
        m.ngroups[m.count] = n[t] / 8;
        if (++m.count == kManyMax) {
            const int rc = flush();
            if (rc) return rc;
        }
    }
    int rc = flush();
    if (rc) return rc;
    for (int t = 0; t < count; ++t) {
        const bool batched = aligned(packed[t], 4) && aligned(out[t], 16) && n[t] >= 8;
        const int64_t start = batched ? n[t] / 8 * 8 : 0;
        if (start >= n[t]) continue;
        dim3 g((unsigned)((n[t] - start + 255) / 256)), b(256);
        if (out_dtype == STM_F16)
            hipLaunchKernelGGL(k_dequantize_generic<STM_F16>, g, b, 0, stream, packed[t], absmax[t], out[t], start,
                               n[t], bshift);
        else if (out_dtype == STM_BF16)
            hipLaunchKernelGGL(k_dequantize_generic<STM_BF16>, g, b, 0, stream, packed[t], absmax[t], out[t], start,
                               n[t], bshift);
        else
            hipLaunchKernelGGL(k_dequantize_generic<STM_F32>, g, b, 0, stream, packed[t], absmax[t], out[t], start,
                               n[t], bshift);
        if ((rc = check_launch("dequantize_many(tail)")) != STM_OK) return rc;
    }
    return STM_OK;
}

}  // namespace stm
