// cpbp_reduce.hip -- CP-BP warp-tile feature-weighted row reduction on gfx950.
//
// Contract (components/CellPack/src/feature_weighted_row_reduction_cuda.cu:180-218):
// for every execution row of every tile, sum over its stored values of
// fp32(value) * w[feature_permutation[block_begin + local]] and write the row's sum to
// row_values[row_permutation[execution_row]] (canonical order). Per row the values are
// visited in the reference's order (descriptor, then local feature), one fp32 FMA each.
//
// Mapping: one wave64 per tile and lane = tile-local row, so a 64-row tile (u64 cell
// masks, the wave64 projection) fills the wavefront; tiles of width <= 32 use u32 masks
// (the reference's v1 contract) with the upper lanes idle. Descriptor fields are
// wave-uniform loads; a lane whose cell bit is set ranks itself among the set bits
// below it (popcount) to find its compacted row-block entry.
#include "cx_common.hpp"

namespace cx {
namespace {

struct CpbpArgs {
    const std::uint32_t *feature_block_offsets;
    const std::uint32_t *feature_permutation;
    const std::uint32_t *tile_block_offsets;
    const std::uint32_t *tile_block_ids;
    const void *cell_masks;
    const std::uint32_t *block_row_entry_offsets;
    const std::uint32_t *gene_masks;
    const std::uint32_t *value_offsets;
    const void *values;
    const std::uint32_t *row_permutation;
    const float *weights;
    float *row_values;
    std::uint32_t row_count;
    std::uint32_t tile_count;
    std::uint32_t tile_row_width;
};

constexpr int kTilesPerBlock = 4;

template<typename MaskT, typename ValT>
__global__ __launch_bounds__(kWave *kTilesPerBlock) void cpbp_reduce_kernel(CpbpArgs a) {
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t tile = blockIdx.x * kTilesPerBlock + threadIdx.x / kWave;
    if (tile >= a.tile_count) return;
    const std::uint32_t exec_row = tile * a.tile_row_width + static_cast<std::uint32_t>(lane);
    const bool active = static_cast<std::uint32_t>(lane) < a.tile_row_width && exec_row < a.row_count;
    const MaskT lane_bit = static_cast<MaskT>(1) << (lane & (sizeof(MaskT) * 8 - 1));
    const MaskT lower = lane_bit - static_cast<MaskT>(1);
    const MaskT *masks = static_cast<const MaskT *>(a.cell_masks);
    const ValT *values = static_cast<const ValT *>(a.values);
    float sum = 0.0f;
    const std::uint32_t d_begin = a.tile_block_offsets[tile];
    const std::uint32_t d_end = a.tile_block_offsets[tile + 1];
    for (std::uint32_t d = d_begin; d < d_end; ++d) {
        const MaskT cell_mask = masks[d];
        if (!active || (cell_mask & lane_bit) == 0) continue;
        const std::uint32_t entry = a.block_row_entry_offsets[d]
            + static_cast<std::uint32_t>(__popcll(static_cast<unsigned long long>(cell_mask & lower)));
        const std::uint32_t block = a.tile_block_ids[d];
        const std::uint32_t block_begin = a.feature_block_offsets[block];
        std::uint32_t gene_mask = a.gene_masks[entry];
        std::uint32_t v = a.value_offsets[entry];
        while (gene_mask != 0u) {
            const std::uint32_t local = static_cast<std::uint32_t>(__builtin_ctz(gene_mask));
            gene_mask &= gene_mask - 1u;
            const std::uint32_t feature = a.feature_permutation[block_begin + local];
            float x;
            if constexpr (sizeof(ValT) == 2) x = h2f(values[v]);
            else x = values[v];
            sum = __builtin_fmaf(x, a.weights[feature], sum);
            ++v;
        }
    }
    if (active) a.row_values[a.row_permutation[exec_row]] = sum;
}

} // namespace
} // namespace cx

extern "C" int cx_cpbp_reduce(const cx_cpbp_tiles *t, const float *feature_weights,
                              uint64_t feature_weight_capacity, float *row_values,
                              uint64_t row_capacity, void *stream) {
    using namespace cx;
    clear_error();
    if (t == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_cpbp_reduce: null tiles");
    // Metadata checks of validate_metadata (feature_weighted_row_reduction_cuda.cu:57-136).
    if (t->value_dtype != CELLERATOR_DTYPE_F16 && t->value_dtype != CELLERATOR_DTYPE_F32)
        return fail(CX_STATUS_UNSUPPORTED, "cx_cpbp_reduce: values must be F16 or F32");
    if (t->tile_row_width == 0u || t->tile_row_width > 64u)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_cpbp_reduce: tile_row_width must be 1..64");
    const std::uint64_t expected_tiles = (static_cast<std::uint64_t>(t->row_count) + t->tile_row_width - 1u)
        / t->tile_row_width;
    if (t->tile_count != expected_tiles || t->tile_block_count > t->row_block_entry_count
        || t->row_block_entry_count > t->nnz_count)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_cpbp_reduce: tile, descriptor or entry counts are inconsistent");
    if (feature_weight_capacity < t->feature_count)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_cpbp_reduce: feature weight capacity is too small");
    if (row_capacity < t->row_count)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_cpbp_reduce: output capacity is insufficient");
    if (t->feature_block_offsets == nullptr
        || (t->feature_count != 0u && (t->feature_permutation == nullptr || feature_weights == nullptr))
        || t->tile_block_offsets == nullptr || t->block_row_entry_offsets == nullptr
        || (t->row_count != 0u && (t->row_permutation == nullptr || row_values == nullptr))
        || (t->tile_block_count != 0u && (t->tile_block_ids == nullptr || t->tile_block_cell_masks == nullptr))
        || (t->row_block_entry_count != 0u
            && (t->row_block_gene_masks == nullptr || t->row_block_value_offsets == nullptr))
        || (t->nnz_count != 0u && t->values == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_cpbp_reduce: device input pointer is null");
    // Output aliasing (validate_output, :138-178).
    const void *inputs[] = {feature_weights, t->feature_block_offsets, t->feature_permutation,
                            t->tile_block_offsets, t->tile_block_ids, t->tile_block_cell_masks,
                            t->block_row_entry_offsets, t->row_block_gene_masks,
                            t->row_block_value_offsets, t->values, t->row_permutation};
    for (const void *p : inputs)
        if (p != nullptr && p == static_cast<const void *>(row_values))
            return fail(CX_STATUS_INVALID_ARGUMENT, "cx_cpbp_reduce: output aliases an input");
    if (t->row_count == 0u) return CX_STATUS_SUCCESS;

    CpbpArgs a{};
    a.feature_block_offsets = t->feature_block_offsets;
    a.feature_permutation = t->feature_permutation;
    a.tile_block_offsets = t->tile_block_offsets;
    a.tile_block_ids = t->tile_block_ids;
    a.cell_masks = t->tile_block_cell_masks;
    a.block_row_entry_offsets = t->block_row_entry_offsets;
    a.gene_masks = t->row_block_gene_masks;
    a.value_offsets = t->row_block_value_offsets;
    a.values = t->values;
    a.row_permutation = t->row_permutation;
    a.weights = feature_weights;
    a.row_values = row_values;
    a.row_count = t->row_count;
    a.tile_count = t->tile_count;
    a.tile_row_width = t->tile_row_width;
    const dim3 grid((t->tile_count + kTilesPerBlock - 1) / kTilesPerBlock), block(kWave * kTilesPerBlock);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool wide = t->tile_row_width > 32u;
    const bool half = t->value_dtype == CELLERATOR_DTYPE_F16;
    if (wide && half) hipLaunchKernelGGL((cpbp_reduce_kernel<std::uint64_t, std::uint16_t>), grid, block, 0, s, a);
    else if (wide) hipLaunchKernelGGL((cpbp_reduce_kernel<std::uint64_t, float>), grid, block, 0, s, a);
    else if (half) hipLaunchKernelGGL((cpbp_reduce_kernel<std::uint32_t, std::uint16_t>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((cpbp_reduce_kernel<std::uint32_t, float>), grid, block, 0, s, a);
    return check_launch("cpbp_reduce");
}
