// Launchers implemented by the kernel translation units.
#pragma once

#include "nf4_common.h"

namespace stm {

// One description for the dense and the grouped (per-expert) GEMMs.
//   forward : out[M, N] = a[M, K] . W[N, K]^T (+ bias) (+ lora_x[M, R] . lora_w[N, R]^T)
//   backward: out[M, K] = a[M, N] . W[N, K]        (+ lora_x[M, R] . lora_w[K, R]^T)
// Grouped: `offsets` (device int32 [num_groups + 1]) splits the rows of a/out by
// expert; expert e uses the e-th [N, K] slice of the stacked NF4 payload and M
// is the largest row count of any expert.
struct GemmArgs {
    const void* a;
    const uint8_t* packed;
    const float* absmax;
    const void* bias;
    const void* lora_x;
    const void* lora_w;
    int lora_rank;
    void* out;
    int64_t M, N, K;
    int blocksize;
    const int32_t* offsets;
    int num_groups;
    // Split reduction: when splits > 1, work-group z of a tile covers reduction
    // steps [z * steps / splits, (z + 1) * steps / splits) and stores its fp32 tile
    // to partial[z][row][col]; a second kernel sums the splits (fixed order),
    // adds the bias and rounds once.
    float* partial;
    int splits;
    // Grouped forward: tile height chosen from the host's per-expert row counts
    // (grouped_tile_rows); 0 = the planner's 256-row tile.
    int group_bm;
    // 1: the register-weight kernels write the output with non-temporal stores.
    // Set for outputs of at least kStreamOutBytes: the next kernel would not
    // find them in the 256 MB infinity cache anyway, and written back later
    // they compete with that kernel's reads (the LoRA step's backward reads dY
    // right after the forward wrote a 235 MB output: 1.2 % per step).
    int stream_out;
};

constexpr int64_t kStreamOutBytes = 64ll << 20;

// Split count the launchers use for a problem (1 = no split) and the fp32
// workspace it needs: sized so that small-M problems still put >= 512
// work-groups (two per CU of MI355X's 256) on the GPU.
int gemm_splits(int64_t M, int64_t N, int64_t K, bool backward, int num_groups);
int64_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, bool backward, int num_groups);

// Restrict the planner to one tile kind (0 = 256 x 256, 1 = 128 x 128,
// 2 = 128 x 256; anything else = the cost model). Returns the previous setting.
int set_gemm_tile(int kind);

// Tile height (192 or 256 rows) of the grouped forward for experts with the
// row counts offsets[e + 1] - offsets[e] (host array of num_experts + 1
// entries): the one that computes the fewest padded rows, a 192-row row
// weighted 8 % dearer (its weights are dequantized for fewer rows).
int grouped_tile_rows(const int32_t* offsets, int num_experts);

int launch_quantize(const void* A, int dtype, int64_t n, int blocksize, const CellTable& tab, uint8_t* packed,
                    float* absmax, hipStream_t stream);
int launch_dequantize(const uint8_t* packed, const float* absmax, int64_t n, int blocksize, void* out, int out_dtype,
                      hipStream_t stream);
// Many tensors of one dtype / blocksize (/ rule): batched launches of whole
// blocks, per-tensor launches for partial blocks and unaligned tensors.
int launch_quantize_many(int count, const void* const* A, const int64_t* n, int dtype, int bs, const CellTable& tab,
                         uint8_t* const* packed, float* const* absmax, hipStream_t stream);
int launch_dequantize_many(int count, const uint8_t* const* packed, const float* const* absmax, const int64_t* n,
                           int bs, void* const* out, int out_dtype, hipStream_t stream);
int launch_gemm_fwd(const GemmArgs& g, int dtype, hipStream_t stream);
int launch_gemm_bwd(const GemmArgs& g, int dtype, hipStream_t stream);

}  // namespace stm
