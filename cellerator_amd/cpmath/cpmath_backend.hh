// CP-Math operation-core backend for the MI355X engine: three native candidates that a
// Cellerator build registers in its candidate_registry
// (include/Cellerator/compute/math/operation_core/operation_core.hh:195-212) and then
// prepares and runs through prepare_candidate / run_prepared_operation
// (src/compute/math/operation_core/operation_core.cc:136-242).
//
//   quantized_csr_candidate                  sparse_dense_multiply    x csr               x native_direct
//   quantized_csr_execution_order_candidate  sparse_dense_multiply    x csr               x native_direct
//   blocked_ell_candidate                    sparse_dense_multiply    x blocked_ell       x native_direct
//   cpbp_candidate                           weighted_relation_reduce x native_row_masked x native_direct
//
// The two quantized CSR candidates compute the same product. The first runs on the CSR as
// bound (the row-group kernel); the second on a prepared execution-order projection of it
// (popularity order, a dense head on the matrix cores and a prepared tail stream, built once by
// prepare_quantized_csr_execution_order and kept as persistent state), which is about twice as
// fast per launch at the benchmark shapes but costs a one-time preparation and persistent
// device memory; the planner weighs the two through their phase costs and the reuse it is told.
//
// This file compiles against the reference's public headers (types and inline validators
// only) and links against libcellerator_amd.so, whose C-ABI (include/cellerator_amd.h)
// launches the HIP kernels. It calls no function of the reference's own libraries.
//
// Flow. The operation core's prepare callback receives keys only, so the axes and shapes
// an operation binds are declared once per projection with declare_projection(); prepare
// finds the declaration by its projection handle and freezes the binding contract from it.
// The prepared_operation borrows that declaration (persistent state): retire it only
// after every prepared operation made from it is gone.
//
// Operands of a launch (execution::launch_bindings, launch_bindings.hh:85-97):
//   inputs[0]  sparse_relation (axes cells x genes). projection_data points to the
//              engine's typed physical view of the structure -- cx_qcsr_matrix,
//              cx_bell_matrix or cx_cpbp_tiles -- with every value pointer NULL, and
//              projection_bytes == sizeof of that view. A CP-BP projection may instead
//              carry the reference's native_tile_view (cx_native_tile_view, same layout,
//              native_tile_view.hh:45-54, built with its sidecars): its compact values must
//              then be the bound value plane's or NULL.
//   values[0]  the value plane of that structure: quantized codes (u8 storage, per-gene
//              affine as quantization_kind::per_module with one group per gene) or plain
//              f16 / bf16 / f32 values.
//   inputs[1]  dense_tensor: W [genes x N] row-major (multiply) or w [genes] (reduce).
//   outputs[0] dense_tensor f32: Y [cells x N] row-major, or y [cells] in canonical order.
// The stream is launch.stream.stream (a hipStream_t, NULL = the null stream). Run
// launches kernels only: it neither allocates, synchronizes nor queries the device.
//
// Fused epilogues (the two multiply candidates). operation_problem names the operation's
// semantics, so an epilogue travels in problem.operation = spmm_operation(kind, affine):
//   kind    the reference's epilogue_kind (operation.hh:49-58, CX_EPILOGUE_*): bias kinds
//           bind inputs[2] = bias, a dense f32 [N] tensor on the output axis
//           (numeric_policy.bias = f32, problem.input_count = 3); the others take none
//           (numeric_policy.bias = invalid, input_count = 2);
//   affine  output effect affine_accumulate: Y = act(alpha * A.W + beta * Y + bias) in
//           place, alpha and beta bound per launch as f32 (or f64) scalars with binding ids
//           alpha_binding and beta_binding. Otherwise the effect is overwrite.
// Any other problem.operation is the plain product (kind none, overwrite).
#pragma once

#include <Cellerator/compute/math/operation_core/operation_core.hh>
#include <Cellerator/planner/end_to_end_planner.hh>

#include <cstdint>

#include "cellerator_amd.h"

namespace cellerator_amd::cpmath {

namespace core = cellerator::compute::math::core;
namespace execution = cellerator::execution;

// projection_key.schema_version of the engine's physical views.
inline constexpr std::uint16_t physical_view_schema = 1u;

// Candidate identities; kernel identities of the prepared dispatch.
inline constexpr core::stable_id quantized_csr_candidate_id{0x4358414d44514353ull, 1u};
inline constexpr core::stable_id quantized_csr_execution_order_candidate_id{0x4358414d44514353ull, 2u};
inline constexpr core::stable_id blocked_ell_candidate_id{0x4358414d4442454cull, 1u};
inline constexpr core::stable_id cpbp_candidate_id{0x4358414d44435042ull, 1u};
inline constexpr core::stable_id blocked_ell_mfma_kernel_id{0x4358414d4442454cull, 2u};
inline constexpr core::stable_id blocked_ell_generic_kernel_id{0x4358414d4442454cull, 3u};

// problem.operation of a multiply with a fused epilogue (see the file comment).
inline constexpr std::uint64_t spmm_epilogue_family = 0x4358414d44455049ull;
inline constexpr std::uint64_t spmm_affine_flag = 0x100u;
inline constexpr std::uint32_t alpha_binding = 0u;
inline constexpr std::uint32_t beta_binding = 1u;

constexpr core::stable_id spmm_operation(std::uint32_t kind, bool affine) noexcept {
    return {spmm_epilogue_family, static_cast<std::uint64_t>(kind) | (affine ? spmm_affine_flag : 0u)};
}

// projection_key.variant of a quantized CSR projection: the code width in bits (1, 2, 4,
// 8), or 0 for plain f16 / f32 values.
//
// What the caller states once per projection.
struct projection_declaration {
    core::projection_key key{};                 // handle, persistent id, kind, schema, variant
    execution::relation_structure structure{};  // source axis = cells, destination = genes
    execution::structure_id persistent_structure{};
    execution::axis_identity output_axis{};     // the N axis of W and Y (multiply only)
    std::uint32_t rows = 0u;                    // cells
    std::uint32_t cols = 0u;                    // genes
    std::uint32_t output_columns = 0u;          // N (multiply); 0 for the reduction
    std::uint32_t block_size = 0u;              // Blocked-ELL block edge; 0 otherwise
    std::uint32_t head_genes = 0u;              // execution-order candidate: genes on the matrix cores, a
                                                // multiple of 1,024 (0: 2,048)
};

core::operation_status declare_projection(const projection_declaration &declaration) noexcept;
core::operation_status retire_projection(execution::projection_handle projection) noexcept;

// Persistent physical state of a declared quantized CSR projection. A one-time preparation,
// not a launch: it enqueues work on `stream` and synchronizes it.
//  * The structure's column order is checked once on the device (cx_qcsr_check_columns).
//    Launches whose sparse view carries that structure (the same row_ptr and col_idx; the
//    core already pins the structure handle and epoch) then run with
//    CX_QCSR_COLUMNS_SORTED, the kernels that skip the per-entry order check.
//  * With `pairs` (device, 2 x genes floats, caller-owned, outliving the projection), the
//    per-gene scales and offsets of `plane` are interleaved into it. Launches whose value
//    plane has the same generation and metadata pointers then decode from the pairs
//    (CX_DECODE_PER_GENE_AFFINE_PAIRS, bit-identical to the separate arrays); any other
//    plane decodes from its own arrays.
// A sparse view's own flags must be 0: only this preparation establishes them.
core::operation_status prepare_quantized_csr_state(execution::projection_handle projection,
                                                   const cx_qcsr_matrix &structure,
                                                   const execution::value_plane *plane,
                                                   float *pairs, void *stream) noexcept;

// Persistent state of the execution-order candidate for a declared quantized CSR projection:
// the engine's prepared execution-order projection (cx_qcsr_exec_prepare) of `structure` with
// the codes and per-gene f32 metadata of `plane`, head width from the declaration. A one-time
// preparation: it allocates the projection's device memory (held until the projection is
// retired or prepared again), enqueues work on `stream` and synchronizes it. Launches of the
// execution-order candidate whose sparse view carries the same structure arrays and whose value
// plane has the same generation, codes and metadata pointers run the prepared path
// (last_dispatch "qcsr:execution-order"); any other launch -- new values, no preparation yet,
// f32 W or an output the prepared path cannot write -- runs the row-group kernel on the bound
// operands ("qcsr:execution-order->row-group"), so results stay correct. Rows may repeat no
// gene (INVALID_ARGUMENT otherwise).
core::operation_status prepare_quantized_csr_execution_order(execution::projection_handle projection,
                                                             const cx_qcsr_matrix &structure,
                                                             const execution::value_plane &plane,
                                                             void *stream) noexcept;
// Device bytes the execution-order state of `projection` holds (0 when none).
std::uint64_t execution_order_persistent_bytes(execution::projection_handle projection) noexcept;

// Persistent state of a declared Blocked-ELL projection for the MFMA kernels (bf16 values
// and weights, 32 x 32 blocks). A one-time preparation that synchronizes `stream`.
//  * `panel` (device, ceil(genes/32) * 32 * N bf16, caller-owned) is packed now from
//    `weights` (device bf16 [genes x N], row stride weights_ld). Launches whose W is that
//    same pointer read the panel instead of repacking W into the workspace. Call again
//    after W is written in place: the panel is the weight generation packed last.
//  * `groups` (cx_bell_plan_groups of this structure, device arrays, caller-owned): launches
//    whose view carries the same block_col_idx run the grouped kernel. NULL keeps the
//    per-row-block kernel.
core::operation_status prepare_blocked_ell_state(execution::projection_handle projection,
                                                 const cx_bell_matrix &structure,
                                                 const uint16_t *weights, int64_t weights_ld,
                                                 uint16_t *panel, const cx_bell_groups *groups,
                                                 void *stream) noexcept;

// The reduction contract of a declared CP-BP projection, checked once (host only):
// cx_cpbp_reduction_validate -- versions, numeric contract, identities including the
// recomputed reduction identity, and the plan / order / tile domains, the checks of the
// reference's validate_metadata (components/CellPack/src/feature_weighted_row_reduction_cuda.cu:57-136).
// After it, a launch runs only if its tile view equals the validated view's tiles
// ("cpbp:checked"); without it the tile view is run as bound ("cpbp:unchecked").
// `entry_rows` (optional, caller-owned device memory of entry_rows_capacity u32, at least
// the tiles' row_block_entry_count; kept until the projection is retired) receives
// cx_cpbp_entry_rows of the validated tiles, enqueued on `stream`; checked launches then
// read each entry's row and block start from it ("cpbp:checked+entry-rows"), bitwise the
// same sums as the descriptor walk.
core::operation_status prepare_cpbp_state(execution::projection_handle projection,
                                          const cx_cpbp_reduction_view &view, uint32_t *entry_rows = nullptr,
                                          uint64_t entry_rows_capacity = 0u, void *stream = nullptr) noexcept;

// Kernel form the last successful run on this thread dispatched, e.g.
// "qcsr:pairs+sorted", "qcsr:gene-affine", "qcsr:execution-order", "bell:grouped+panel",
// "bell:mfma+repack", "bell:generic", "cpbp:checked", "cpbp:checked+entry-rows",
// "cpbp:native-tile".
const char *last_dispatch() noexcept;

core::operation_candidate quantized_csr_candidate() noexcept;
core::operation_candidate quantized_csr_execution_order_candidate() noexcept;
core::operation_candidate blocked_ell_candidate() noexcept;
core::operation_candidate cpbp_candidate() noexcept;

// Engine error text behind the last execution_failed status of this thread.
const char *last_engine_error() noexcept;

// ---- planner side (include/Cellerator/planner/end_to_end_planner.hh:118-291) ----------
// What an end-to-end planner needs to rank the engine's candidates without running them:
// the shape of the work and an analytical cost per phase from MI355X peaks (HBM 8 TB/s,
// non-packed fp32 VALU 78.6 TFLOP/s, bf16 matrix cores 2.5 PFLOP/s) scaled by the fraction
// of peak each kernel family reaches, and the physical bytes each projection keeps. The
// planner's measurement hook then replaces the kernel estimate with timings of the real
// kernels.
struct workload_shape {
    std::uint64_t rows = 0u;          // cells
    std::uint64_t cols = 0u;          // genes
    std::uint64_t nnz = 0u;           // stored entries of the logical matrix
    std::uint32_t out_cols = 0u;      // N (multiply); 0 for the reduction
    std::uint32_t bits = 0u;          // quantized code width; 0 = plain values
    std::uint32_t value_bytes = 4u;   // bytes per plain value (Blocked-ELL, CP-BP)
    std::uint32_t block_size = 0u;    // Blocked-ELL block edge
    std::uint64_t ell_columns = 0u;   // Blocked-ELL padded columns per row
    std::uint64_t tile_blocks = 0u;   // CP-BP (tile, block) entries
    std::uint32_t head_genes = 0u;    // execution-order quantized CSR: matrix-core head width (0: 2,048)
    std::uint32_t reserved = 0u;
};

// Analytical phases of `candidate` (one of the three above) on `shape`; false for an
// unknown candidate or an incomplete shape.
bool analytical_costs(core::stable_id candidate, const workload_shape &shape,
                      cellerator::planner::phase_costs *out) noexcept;
// A planner candidate for an engine operation candidate and its declared projection:
// identity and name of the operation candidate, flags from its capabilities (correct by
// construction, deterministic and graph capture as advertised), analytical phases.
bool planner_candidate_for(const core::operation_candidate &operation, const core::projection_key &projection,
                           const workload_shape &shape, cellerator::planner::planner_candidate *out) noexcept;

} // namespace cellerator_amd::cpmath
