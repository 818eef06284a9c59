// SwiGLU gating of a frozen MLP (gfx950), the elementwise step between the
// stacked gate/up projection and the down projection:
//
//   forward   h[r, i]  = silu(g) * u,           g = gu[r, i], u = gu[r, I + i]
//   backward  dg[r, i] = dh * u * silu'(g),     du[r, i] = dh * silu(g)
//             silu(g) = g * s, silu'(g) = s * (1 + g * (1 - s)), s = 1 / (1 + exp(-g))
//
// gu is the output of the stacked [gate; up] projection, one row [g_0..g_I-1,
// u_0..u_I-1] per token; dgu has the same layout, so the input gradient of both
// projections is one GEMM against the same stacked weight. Arithmetic is fp32
// with one round-to-nearest-even conversion per output.
//
// Memory-bound: forward moves 6 bytes per h element (g, u in; h out), backward
// 10 (dh, g, u in; dg, du out). Each lane handles 8 consecutive columns with
// 16-byte accesses; rows whose width is not a multiple of 8 go through a scalar
// kernel.
#include "nf4_common.h"

namespace stm {
namespace {

__device__ __forceinline__ float sigmoid(float g) { return 1.0f / (1.0f + expf(-g)); }

template <typename Tr>
__device__ __forceinline__ void unpack8(const uint4& v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = Tr::to_f32((uint16_t)(w[i] & 0xFFFFu));
        f[2 * i + 1] = Tr::to_f32((uint16_t)(w[i] >> 16));
    }
}

template <typename Tr>
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
    return make_uint4(Tr::pack2(f[0], f[1]), Tr::pack2(f[2], f[3]), Tr::pack2(f[4], f[5]), Tr::pack2(f[6], f[7]));
}

template <typename Tr>
__global__ __launch_bounds__(256) void k_swiglu_fwd(const uint16_t* __restrict__ gu, uint16_t* __restrict__ h,
                                                    int64_t rows, int64_t inter) {
    const int64_t vpr = inter / 8;  // 8-column vectors per row
    const int64_t total = rows * vpr;
    for (int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; v < total; v += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = v / vpr, c = (v - r * vpr) * 8;
        const uint16_t* row = gu + r * 2 * inter;
        float g[8], u[8], o[8];
        unpack8<Tr>(*reinterpret_cast<const uint4*>(row + c), g);
        unpack8<Tr>(*reinterpret_cast<const uint4*>(row + inter + c), u);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = g[i] * sigmoid(g[i]) * u[i];
        *reinterpret_cast<uint4*>(h + r * inter + c) = pack8<Tr>(o);
    }
}

template <typename Tr>
__global__ __launch_bounds__(256) void k_swiglu_bwd(const uint16_t* __restrict__ dh, const uint16_t* __restrict__ gu,
                                                    uint16_t* __restrict__ dgu, int64_t rows, int64_t inter) {
    const int64_t vpr = inter / 8;
    const int64_t total = rows * vpr;
    for (int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; v < total; v += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = v / vpr, c = (v - r * vpr) * 8;
        const uint16_t* row = gu + r * 2 * inter;
        float g[8], u[8], d[8], dg[8], du[8];
        unpack8<Tr>(*reinterpret_cast<const uint4*>(row + c), g);
        unpack8<Tr>(*reinterpret_cast<const uint4*>(row + inter + c), u);
        unpack8<Tr>(*reinterpret_cast<const uint4*>(dh + r * inter + c), d);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float s = sigmoid(g[i]);
            du[i] = d[i] * (g[i] * s);
            dg[i] = d[i] * u[i] * (s * (1.0f + g[i] * (1.0f - s)));
        }
        uint16_t* orow = dgu + r * 2 * inter;
        *reinterpret_cast<uint4*>(orow + c) = pack8<Tr>(dg);
        *reinterpret_cast<uint4*>(orow + inter + c) = pack8<Tr>(du);
    }
}

// Scalar forms for widths that are not a multiple of 8 or unaligned buffers.
template <typename Tr>
__global__ __launch_bounds__(256) void k_swiglu_fwd_scalar(const uint16_t* __restrict__ gu, uint16_t* __restrict__ h,
                                                           int64_t rows, int64_t inter) {
    const int64_t total = rows * inter;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / inter, c = e - r * inter;
        const float g = Tr::to_f32(gu[r * 2 * inter + c]), u = Tr::to_f32(gu[r * 2 * inter + inter + c]);
        h[e] = Tr::from_f32(g * sigmoid(g) * u);
    }
}

template <typename Tr>
__global__ __launch_bounds__(256) void k_swiglu_bwd_scalar(const uint16_t* __restrict__ dh,
                                                           const uint16_t* __restrict__ gu, uint16_t* __restrict__ dgu,
                                                           int64_t rows, int64_t inter) {
    const int64_t total = rows * inter;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / inter, c = e - r * inter;
        const float g = Tr::to_f32(gu[r * 2 * inter + c]), u = Tr::to_f32(gu[r * 2 * inter + inter + c]);
        const float d = Tr::to_f32(dh[e]), s = sigmoid(g);
        dgu[r * 2 * inter + c] = Tr::from_f32(d * u * (s * (1.0f + g * (1.0f - s))));
        dgu[r * 2 * inter + inter + c] = Tr::from_f32(d * (g * s));
    }
}

unsigned grid_for(int64_t items) {
    const int64_t blocks = (items + 255) / 256;
    return (unsigned)(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

// Empty problems (rows or inter 0) are valid with any pointers, null included.
int check_args(const char* what, const void* a, const void* b, const void* c, int64_t rows, int64_t inter, int dtype) {
    if (rows < 0 || inter < 0) return set_error(STM_ERR_INVALID, "%s: negative size", what);
    if (dtype != STM_BF16 && dtype != STM_F16) return set_error(STM_ERR_INVALID, "%s: dtype must be bf16 or fp16", what);
    if (rows && inter && (!a || !b || !c)) return set_error(STM_ERR_INVALID, "%s: null pointer", what);
    return STM_OK;
}

bool vec_ok(int64_t inter, const void* a, const void* b, const void* c = nullptr) {
    auto al = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; };
    return inter % 8 == 0 && al(a) && al(b) && al(c);
}

}  // namespace
}  // namespace stm

using namespace stm;

extern "C" int stm_swiglu_fwd(const void* gate_up, void* out, int64_t rows, int64_t inter, int dtype, void* stream) {
    int rc = check_args("swiglu_fwd", gate_up, out, out, rows, inter, dtype);
    if (rc) return rc;
    if (rows == 0 || inter == 0) return STM_OK;
    hipStream_t st = (hipStream_t)stream;
    const uint16_t* gu = (const uint16_t*)gate_up;
    uint16_t* h = (uint16_t*)out;
    if (vec_ok(inter, gate_up, out)) {
        const unsigned grid = grid_for(rows * (inter / 8));
        if (dtype == STM_BF16)
            hipLaunchKernelGGL(k_swiglu_fwd<BF16>, dim3(grid), dim3(256), 0, st, gu, h, rows, inter);
        else
            hipLaunchKernelGGL(k_swiglu_fwd<F16>, dim3(grid), dim3(256), 0, st, gu, h, rows, inter);
    } else {
        const unsigned grid = grid_for(rows * inter);
        if (dtype == STM_BF16)
            hipLaunchKernelGGL(k_swiglu_fwd_scalar<BF16>, dim3(grid), dim3(256), 0, st, gu, h, rows, inter);
        else
            hipLaunchKernelGGL(k_swiglu_fwd_scalar<F16>, dim3(grid), dim3(256), 0, st, gu, h, rows, inter);
    }
    return check_launch("swiglu_fwd");
}

extern "C" int stm_swiglu_bwd(const void* grad_out, const void* gate_up, void* grad_gate_up, int64_t rows,
                              int64_t inter, int dtype, void* stream) {
    int rc = check_args("swiglu_bwd", grad_out, gate_up, grad_gate_up, rows, inter, dtype);
    if (rc) return rc;
    if (rows == 0 || inter == 0) return STM_OK;
    hipStream_t st = (hipStream_t)stream;
    const uint16_t* dh = (const uint16_t*)grad_out;
    const uint16_t* gu = (const uint16_t*)gate_up;
    uint16_t* dgu = (uint16_t*)grad_gate_up;
    if (vec_ok(inter, grad_out, gate_up, grad_gate_up)) {
        const unsigned grid = grid_for(rows * (inter / 8));
        if (dtype == STM_BF16)
            hipLaunchKernelGGL(k_swiglu_bwd<BF16>, dim3(grid), dim3(256), 0, st, dh, gu, dgu, rows, inter);
        else
            hipLaunchKernelGGL(k_swiglu_bwd<F16>, dim3(grid), dim3(256), 0, st, dh, gu, dgu, rows, inter);
    } else {
        const unsigned grid = grid_for(rows * inter);
        if (dtype == STM_BF16)
            hipLaunchKernelGGL(k_swiglu_bwd_scalar<BF16>, dim3(grid), dim3(256), 0, st, dh, gu, dgu, rows, inter);
        else
            hipLaunchKernelGGL(k_swiglu_bwd_scalar<F16>, dim3(grid), dim3(256), 0, st, dh, gu, dgu, rows, inter);
    }
    return check_launch("swiglu_bwd");
}
