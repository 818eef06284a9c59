// extern "C" entry points of libstratum_nf4.so: argument validation, error
// reporting, the decision-boundary tables, and dispatch to the kernels.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "nf4_common.h"
#include "nf4_kernels.h"

namespace stm {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(STM_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return STM_OK;
}

// ---------------------------------------------------------------- boundaries
// fp32 values ordered as integers (monotone in the float order, -0 == +0 side by side).
static int64_t fkey(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (u & 0x80000000u) ? -(int64_t)(u & 0x7FFFFFFFu) : (int64_t)u;
}
static float from_key(int64_t k) {
    uint32_t u = k >= 0 ? (uint32_t)k : (0x80000000u | (uint32_t)(-k));
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// argmin rule between level i and i+1: level i+1 wins iff its fp32 distance is strictly smaller.
static bool upper_wins(float s, int i) { return fabsf(s - kLevelsHost[i + 1]) < fabsf(s - kLevelsHost[i]); }

int decision_boundaries(int rounding, float out[15]) {
    for (int i = 0; i < 15; ++i) {
        if (rounding == STM_NF4_THRESHOLD) {
            float t = (float)(((double)kLevelsHost[i] + (double)kLevelsHost[i + 1]) * 0.5);
            out[i] = nextafterf(t, INFINITY);  // s > t  <=>  s >= next(t)
        } else if (rounding == STM_NF4_ARGMIN) {
            int64_t lo = fkey(kLevelsHost[i]), hi = fkey(kLevelsHost[i + 1]);  // P(lo) false, P(hi) true
            while (hi - lo > 1) {
                int64_t mid = lo + (hi - lo) / 2;
                if (upper_wins(from_key(mid), i))
                    hi = mid;
                else
                    lo = mid;
            }
            out[i] = from_key(hi);
        } else {
            return set_error(STM_ERR_INVALID, "unknown rounding rule %d", rounding);
        }
    }
    return STM_OK;
}

int build_cell_table(int rounding, CellTable* tab) {
    float b[15];
    int rc = decision_boundaries(rounding, b);
    if (rc) return rc;
    for (int j = 0; j <= 64; ++j) {
        // s values that can land in cell j -- round(128 c + 128) in [4 j, 4 j + 3],
        // i.e. c in [(4 j - 0.5) / 128 - 1, (4 j + 3.5) / 128 - 1] -- widened to a
        // quarter cell on both sides; a boundary in the margin is still exact
        // (every c of the cell is then on one side of it)
        double lo = (j - 0.25) / 32.0 - 1.0, hi = (j + 1.25) / 32.0 - 1.0;
        uint32_t base = 0;
        int inside = 0;
        float bound = 2.0f;  // never reached: clamped s <= 1
        for (int i = 0; i < 15; ++i) {
            if ((double)b[i] <= lo)
                ++base;
            else if ((double)b[i] <= hi) {
                ++inside;
                bound = b[i];
            }
        }
        if (inside > 1) return set_error(STM_ERR_INVALID, "cell %d holds %d boundaries", j, inside);
        tab->bound[j] = bound;
        tab->base[j] = base;
    }
    return STM_OK;
}

// Both rules' tables, built once on first use (a function-local static: its
// initialisation is thread-safe, so concurrent first calls see a finished table).
struct CellTables {
    CellTable tab[2];
    bool ok[2];
    CellTables() {
        for (int r = 0; r < 2; ++r) ok[r] = build_cell_table(r, &tab[r]) == STM_OK;
    }
};

static const CellTable* cell_table(int rounding) {
    static const CellTables tables;
    if (rounding < 0 || rounding > 1 || !tables.ok[rounding]) return nullptr;
    return &tables.tab[rounding];
}

static bool is_16bit(int dt) { return dt == STM_F16 || dt == STM_BF16; }
static bool valid_dtype(int dt) { return dt == STM_F16 || dt == STM_BF16 || dt == STM_F32; }
static bool valid_blocksize(int bs) { return bs >= 64 && bs <= 4096 && is_pow2(bs); }

// ------------------------------------------------- allocation-free scratch
// Device memory of stm_nf4_gemm_fwd_noalloc: the fp32 split-reduction partials
// that stm_nf4_gemm_fwd takes from the caller's workspace. One array per GPU
// (each device holds its own copy of a __device__ variable, for the life of
// the process). In host code `scratch` names a host-side stand-in, not a
// device address: kernels receive the per-device address that
// hipGetSymbolAddress returns, fetched once per device.
constexpr int64_t kScratchBytes = (int64_t)16 << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// The scratch address on the current device (fetched on the first call there).
static int scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(STM_ERR_HIP, "gemm_fwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return set_error(STM_ERR_UNSUPPORTED, "gemm_fwd_noalloc: device %d", dev);
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p)
                return set_error(STM_ERR_HIP, "gemm_fwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                                 hipGetErrorString(e));
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return STM_OK;
}

}  // namespace stm

using namespace stm;

extern "C" {

int stm_nf4_abi_version(void) { return STM_NF4_ABI_VERSION; }

const char* stm_last_error(void) { return g_err; }

int stm_nf4_decision_boundaries(int rounding, float* out15) {
    if (!out15) return set_error(STM_ERR_INVALID, "out15 is NULL");
    return decision_boundaries(rounding, out15);
}

int stm_nf4_cell_table(int rounding, float* bound65, uint8_t* base65) {
    if (!bound65 || !base65) return set_error(STM_ERR_INVALID, "NULL output");
    const CellTable* t = cell_table(rounding);
    if (!t) return set_error(STM_ERR_INVALID, "unknown rounding rule %d", rounding);
    for (int j = 0; j < 65; ++j) {
        bound65[j] = t->bound[j];
        base65[j] = (uint8_t)t->base[j];
    }
    return STM_OK;
}

int stm_nf4_quantize(const void* A, int dtype, int64_t n, int blocksize, int rounding, uint8_t* packed,
                     float* absmax, void* stream) {
    g_err[0] = 0;
    if (n < 0) return set_error(STM_ERR_INVALID, "quantize: n = %lld < 0", (long long)n);
    if (!valid_dtype(dtype)) return set_error(STM_ERR_INVALID, "quantize: bad dtype %d", dtype);
    if (!valid_blocksize(blocksize))
        return set_error(STM_ERR_INVALID, "quantize: blocksize %d not a power of two in [64, 4096]", blocksize);
    const CellTable* tab = cell_table(rounding);
    if (!tab) return set_error(STM_ERR_INVALID, "quantize: unknown rounding rule %d", rounding);
    if (n == 0) return STM_OK;
    if (!A || !packed || !absmax) return set_error(STM_ERR_INVALID, "quantize: NULL pointer");
    return launch_quantize(A, dtype, n, blocksize, *tab, packed, absmax, (hipStream_t)stream);
}

int stm_nf4_dequantize(const uint8_t* packed, const float* absmax, int64_t n, int blocksize, void* out,
                       int out_dtype, void* stream) {
    g_err[0] = 0;
    if (n < 0) return set_error(STM_ERR_INVALID, "dequantize: n = %lld < 0", (long long)n);
    if (!valid_dtype(out_dtype)) return set_error(STM_ERR_INVALID, "dequantize: bad dtype %d", out_dtype);
    if (!valid_blocksize(blocksize))
        return set_error(STM_ERR_INVALID, "dequantize: blocksize %d not a power of two in [64, 4096]", blocksize);
    if (n == 0) return STM_OK;
    if (!packed || !absmax || !out) return set_error(STM_ERR_INVALID, "dequantize: NULL pointer");
    return launch_dequantize(packed, absmax, n, blocksize, out, out_dtype, (hipStream_t)stream);
}

int stm_nf4_quantize_many(int count, const void* const* A, const int64_t* n, int dtype, int blocksize, int rounding,
                          uint8_t* const* packed, float* const* absmax, void* stream) {
    g_err[0] = 0;
    if (count < 0) return set_error(STM_ERR_INVALID, "quantize_many: count %d < 0", count);
    if (!valid_dtype(dtype)) return set_error(STM_ERR_INVALID, "quantize_many: bad dtype %d", dtype);
    if (!valid_blocksize(blocksize))
        return set_error(STM_ERR_INVALID, "quantize_many: blocksize %d not a power of two in [64, 4096]", blocksize);
    const CellTable* tab = cell_table(rounding);
    if (!tab) return set_error(STM_ERR_INVALID, "quantize_many: unknown rounding rule %d", rounding);
    if (count == 0) return STM_OK;
    if (!A || !n || !packed || !absmax) return set_error(STM_ERR_INVALID, "quantize_many: NULL array");
    for (int t = 0; t < count; ++t) {
        if (n[t] < 0) return set_error(STM_ERR_INVALID, "quantize_many: n[%d] = %lld < 0", t, (long long)n[t]);
        if (n[t] > 0 && (!A[t] || !packed[t] || !absmax[t]))
            return set_error(STM_ERR_INVALID, "quantize_many: NULL pointer for tensor %d", t);
        if ((n[t] + 3) / 4 > 0x7FFFFFFFLL) return set_error(STM_ERR_UNSUPPORTED, "quantize_many: n[%d] too large", t);
    }
    return launch_quantize_many(count, A, n, dtype, blocksize, *tab, packed, absmax, (hipStream_t)stream);
}

int stm_nf4_dequantize_many(int count, const uint8_t* const* packed, const float* const* absmax, const int64_t* n,
                            int blocksize, void* const* out, int out_dtype, void* stream) {
    g_err[0] = 0;
    if (count < 0) return set_error(STM_ERR_INVALID, "dequantize_many: count %d < 0", count);
    if (!valid_dtype(out_dtype)) return set_error(STM_ERR_INVALID, "dequantize_many: bad dtype %d", out_dtype);
    if (!valid_blocksize(blocksize))
        return set_error(STM_ERR_INVALID, "dequantize_many: blocksize %d not a power of two in [64, 4096]", blocksize);
    if (count == 0) return STM_OK;
    if (!packed || !absmax || !n || !out) return set_error(STM_ERR_INVALID, "dequantize_many: NULL array");
    for (int t = 0; t < count; ++t) {
        if (n[t] < 0) return set_error(STM_ERR_INVALID, "dequantize_many: n[%d] = %lld < 0", t, (long long)n[t]);
        if (n[t] > 0 && (!packed[t] || !absmax[t] || !out[t]))
            return set_error(STM_ERR_INVALID, "dequantize_many: NULL pointer for tensor %d", t);
        if ((n[t] + 255) / 256 > 0x7FFFFFFFLL)
            return set_error(STM_ERR_UNSUPPORTED, "dequantize_many: n[%d] too large", t);
    }
    return launch_dequantize_many(count, packed, absmax, n, blocksize, out, out_dtype, (hipStream_t)stream);
}

static int check_gemm_common(const char* who, const void* a, const uint8_t* packed, const float* absmax,
                             const void* out, int64_t M, int64_t N, int64_t K, int blocksize, int dtype) {
    if (!is_16bit(dtype)) return set_error(STM_ERR_INVALID, "%s: dtype %d is not bf16/fp16", who, dtype);
    if (M < 0 || N < 0 || K < 0) return set_error(STM_ERR_INVALID, "%s: negative size", who);
    if (!valid_blocksize(blocksize)) return set_error(STM_ERR_INVALID, "%s: bad blocksize %d", who, blocksize);
    if (K % 64 != 0 || K % blocksize != 0)
        return set_error(STM_ERR_UNSUPPORTED, "%s: K = %lld must be a multiple of 64 and of blocksize %d", who,
                         (long long)K, blocksize);
    if (M == 0 || N == 0) return STM_OK;
    if (!a || !packed || !absmax || !out) return set_error(STM_ERR_INVALID, "%s: NULL pointer", who);
    if (!aligned(a, 16) || !aligned(out, 16) || !aligned(packed, 16) || !aligned(absmax, 4))
        return set_error(STM_ERR_INVALID, "%s: operands must be 16-byte aligned", who);
    return 1;  // proceed
}

// Non-NULL workspace: at least the bytes stm_nf4_gemm_workspace_bytes reports.
static int check_workspace(const char* who, void* workspace, int64_t workspace_bytes, int64_t need) {
    if (!workspace || need == 0) return STM_OK;
    if (workspace_bytes < need)
        return set_error(STM_ERR_INVALID, "%s: workspace of %lld bytes, %lld needed", who, (long long)workspace_bytes,
                         (long long)need);
    if (!aligned(workspace, 16)) return set_error(STM_ERR_INVALID, "%s: workspace must be 16-byte aligned", who);
    return STM_OK;
}

int stm_nf4_gemm_set_tile(int kind) { return set_gemm_tile(kind); }

int64_t stm_nf4_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int backward) {
    g_err[0] = 0;
    if (M < 0 || N < 0 || K < 0) return set_error(STM_ERR_INVALID, "gemm_workspace_bytes: negative size");
    return gemm_workspace_bytes(M, N, K, backward != 0, 1);
}

int stm_nf4_gemm_fwd(const void* X, const uint8_t* packed, const float* absmax, const void* bias, const void* T,
                     const void* L, int lora_rank, void* Y, int64_t M, int64_t N, int64_t K, int blocksize,
                     int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    int rc = check_gemm_common("gemm_fwd", X, packed, absmax, Y, M, N, K, blocksize, dtype);
    if (rc <= 0) return rc;
    if (N % 8 != 0) return set_error(STM_ERR_UNSUPPORTED, "gemm_fwd: N = %lld must be a multiple of 8", (long long)N);
    if (lora_rank < 0 || lora_rank % 16 != 0 || lora_rank > 256)
        return set_error(STM_ERR_INVALID, "gemm_fwd: lora_rank %d must be a multiple of 16 in [0, 256]", lora_rank);
    if (lora_rank > 0 && (!T || !L || !aligned(T, 16) || !aligned(L, 16)))
        return set_error(STM_ERR_INVALID, "gemm_fwd: lora_rank > 0 needs 16-byte aligned T and L");
    if (bias && !aligned(bias, 2)) return set_error(STM_ERR_INVALID, "gemm_fwd: misaligned bias");
    const int64_t need = gemm_workspace_bytes(M, N, K, false, 1);
    if ((rc = check_workspace("gemm_fwd", workspace, workspace_bytes, need)) != STM_OK) return rc;
    GemmArgs g{};
    g.a = X; g.packed = packed; g.absmax = absmax; g.bias = bias; g.lora_x = lora_rank ? T : nullptr;
    g.lora_w = lora_rank ? L : nullptr; g.lora_rank = lora_rank; g.out = Y; g.M = M; g.N = N; g.K = K;
    g.blocksize = blocksize; g.offsets = nullptr; g.num_groups = 1;
    g.partial = need ? (float*)workspace : nullptr;
    g.stream_out = M * N * 2 >= kStreamOutBytes;
    return launch_gemm_fwd(g, dtype, (hipStream_t)stream);
}

int stm_nf4_gemm_fwd_noalloc(const void* X, const uint8_t* packed, const float* absmax, const void* bias,
                             const void* T, const void* L, int lora_rank, void* Y, int64_t M, int64_t N, int64_t K,
                             int blocksize, int dtype, void* stream) {
    g_err[0] = 0;
    int rc = check_gemm_common("gemm_fwd_noalloc", X, packed, absmax, Y, M, N, K, blocksize, dtype);
    if (rc <= 0) return rc;
    if (N % 8 != 0)
        return set_error(STM_ERR_UNSUPPORTED, "gemm_fwd_noalloc: N = %lld must be a multiple of 8", (long long)N);
    if (lora_rank < 0 || lora_rank % 16 != 0 || lora_rank > 256)
        return set_error(STM_ERR_INVALID, "gemm_fwd_noalloc: lora_rank %d must be a multiple of 16 in [0, 256]",
                         lora_rank);
    if (lora_rank > 0 && (!T || !L || !aligned(T, 16) || !aligned(L, 16)))
        return set_error(STM_ERR_INVALID, "gemm_fwd_noalloc: lora_rank > 0 needs 16-byte aligned T and L");
    if (bias && !aligned(bias, 2)) return set_error(STM_ERR_INVALID, "gemm_fwd_noalloc: misaligned bias");
    const int64_t need = gemm_workspace_bytes(M, N, K, false, 1);
    if (need > kScratchBytes)
        return set_error(STM_ERR_UNSUPPORTED,
                         "gemm_fwd_noalloc: this %lld x %lld x %lld problem splits its reduction into %lld bytes of "
                         "partials, more than the %lld-byte static scratch; call stm_nf4_gemm_fwd with a workspace",
                         (long long)M, (long long)N, (long long)K, (long long)need, (long long)kScratchBytes);
    void* ws = nullptr;
    if (need > 0 && (rc = scratch_address(&ws)) != STM_OK) return rc;
    GemmArgs g{};
    g.a = X; g.packed = packed; g.absmax = absmax; g.bias = bias; g.lora_x = lora_rank ? T : nullptr;
    g.lora_w = lora_rank ? L : nullptr; g.lora_rank = lora_rank; g.out = Y; g.M = M; g.N = N; g.K = K;
    g.blocksize = blocksize; g.offsets = nullptr; g.num_groups = 1;
    g.partial = need ? (float*)ws : nullptr;
    g.stream_out = M * N * 2 >= kStreamOutBytes;
    return launch_gemm_fwd(g, dtype, (hipStream_t)stream);
}

int stm_nf4_gemm_bwd_dx(const void* dY, const uint8_t* packed, const float* absmax, const void* U, const void* At,
                        int lora_rank, void* dX, int64_t M, int64_t N, int64_t K, int blocksize, int dtype,
                        void* workspace, int64_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    int rc = check_gemm_common("gemm_bwd_dx", dY, packed, absmax, dX, M, N, K, blocksize, dtype);
    if (rc <= 0) return rc;
    if (N % 64 != 0)
        return set_error(STM_ERR_UNSUPPORTED, "gemm_bwd_dx: N = %lld must be a multiple of 64", (long long)N);
    if (lora_rank < 0 || lora_rank % 16 != 0 || lora_rank > 256)
        return set_error(STM_ERR_INVALID, "gemm_bwd_dx: lora_rank %d must be a multiple of 16 in [0, 256]",
                         lora_rank);
    if (lora_rank > 0 && (!U || !At || !aligned(U, 16) || !aligned(At, 16)))
        return set_error(STM_ERR_INVALID, "gemm_bwd_dx: lora_rank > 0 needs 16-byte aligned U and At");
    const int64_t need = gemm_workspace_bytes(M, N, K, true, 1);
    if ((rc = check_workspace("gemm_bwd_dx", workspace, workspace_bytes, need)) != STM_OK) return rc;
    GemmArgs g{};
    g.a = dY; g.packed = packed; g.absmax = absmax; g.bias = nullptr; g.lora_x = lora_rank ? U : nullptr;
    g.lora_w = lora_rank ? At : nullptr; g.lora_rank = lora_rank; g.out = dX; g.M = M; g.N = N; g.K = K;
    g.blocksize = blocksize; g.offsets = nullptr; g.num_groups = 1;
    g.partial = need ? (float*)workspace : nullptr;
    g.stream_out = M * K * 2 >= kStreamOutBytes;
    return launch_gemm_bwd(g, dtype, (hipStream_t)stream);
}

// Host copy of a grouped call's expert offsets: offsets[0] = 0, non-decreasing,
// and (max_rows >= 0) no expert above max_rows rows. Read entirely on the host,
// before any launch.
static int check_host_offsets(const char* fn, const int32_t* h, int num_experts, int64_t max_rows) {
    if (h[0] != 0) return set_error(STM_ERR_INVALID, "%s: offsets[0] = %d, expected 0", fn, h[0]);
    for (int e = 0; e < num_experts; ++e) {
        const int64_t rows = (int64_t)h[e + 1] - h[e];
        if (rows < 0)
            return set_error(STM_ERR_INVALID, "%s: offsets decrease at expert %d (%d -> %d)", fn, e, h[e], h[e + 1]);
        if (max_rows >= 0 && rows > max_rows)
            return set_error(STM_ERR_INVALID, "%s: expert %d has %lld rows, above max_rows %lld", fn, e,
                             (long long)rows, (long long)max_rows);
    }
    return STM_OK;
}

int stm_nf4_grouped_tile_rows(const int32_t* host_offsets, int num_experts) {
    g_err[0] = 0;
    if (!host_offsets || num_experts <= 0)
        return set_error(STM_ERR_INVALID, "grouped_tile_rows: NULL offsets or num_experts %d", num_experts);
    const int rc = check_host_offsets("grouped_tile_rows", host_offsets, num_experts, -1);
    if (rc != STM_OK) return rc;
    return grouped_tile_rows(host_offsets, num_experts);
}

int stm_nf4_grouped_gemm_fwd(const void* X, const uint8_t* packed, const float* absmax, const int32_t* offsets,
                             const int32_t* host_offsets, int num_experts, int64_t max_rows, void* Y, int64_t N,
                             int64_t K, int blocksize, int dtype, void* stream) {
    g_err[0] = 0;
    if (num_experts <= 0 || max_rows < 0)
        return set_error(STM_ERR_INVALID, "grouped_gemm_fwd: num_experts %d, max_rows %lld", num_experts,
                         (long long)max_rows);
    int rc = check_gemm_common("grouped_gemm_fwd", X, packed, absmax, Y, max_rows, N, K, blocksize, dtype);
    if (rc <= 0) return rc;
    if (!offsets) return set_error(STM_ERR_INVALID, "grouped_gemm_fwd: NULL offsets");
    if (N % 8 != 0) return set_error(STM_ERR_UNSUPPORTED, "grouped_gemm_fwd: N must be a multiple of 8");
    if (host_offsets && (rc = check_host_offsets("grouped_gemm_fwd", host_offsets, num_experts, max_rows)) != STM_OK)
        return rc;
    GemmArgs g{};
    g.a = X; g.packed = packed; g.absmax = absmax; g.out = Y; g.M = max_rows; g.N = N; g.K = K;
    g.blocksize = blocksize; g.offsets = offsets; g.num_groups = num_experts;
    g.group_bm = host_offsets ? grouped_tile_rows(host_offsets, num_experts) : 0;
    g.stream_out = host_offsets && (int64_t)host_offsets[num_experts] * N * 2 >= kStreamOutBytes;
    return launch_gemm_fwd(g, dtype, (hipStream_t)stream);
}

int stm_nf4_grouped_gemm_bwd_dx(const void* dY, const uint8_t* packed, const float* absmax, const int32_t* offsets,
                                const int32_t* host_offsets, int num_experts, int64_t max_rows, void* dX, int64_t N,
                                int64_t K, int blocksize, int dtype, void* stream) {
    g_err[0] = 0;
    if (num_experts <= 0 || max_rows < 0)
        return set_error(STM_ERR_INVALID, "grouped_gemm_bwd_dx: num_experts %d, max_rows %lld", num_experts,
                         (long long)max_rows);
    int rc = check_gemm_common("grouped_gemm_bwd_dx", dY, packed, absmax, dX, max_rows, N, K, blocksize, dtype);
    if (rc <= 0) return rc;
    if (!offsets) return set_error(STM_ERR_INVALID, "grouped_gemm_bwd_dx: NULL offsets");
    if (N % 64 != 0) return set_error(STM_ERR_UNSUPPORTED, "grouped_gemm_bwd_dx: N must be a multiple of 64");
    if (host_offsets &&
        (rc = check_host_offsets("grouped_gemm_bwd_dx", host_offsets, num_experts, max_rows)) != STM_OK)
        return rc;
    GemmArgs g{};
    g.a = dY; g.packed = packed; g.absmax = absmax; g.out = dX; g.M = max_rows; g.N = N; g.K = K;
    g.blocksize = blocksize; g.offsets = offsets; g.num_groups = num_experts;
    g.stream_out = host_offsets && (int64_t)host_offsets[num_experts] * K * 2 >= kStreamOutBytes;
    return launch_gemm_bwd(g, dtype, (hipStream_t)stream);
}

}  // extern "C"
