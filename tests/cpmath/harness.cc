// Test harness: drives the engine's CP-Math candidates through the reference's own
// operation core (src/compute/math/operation_core/operation_core.cc, compiled from its
// source into oracle/_ref/ by oracle/Makefile), the way a Cellerator host would:
// register_candidate -> find_candidate -> prepare_candidate -> run_prepared_operation
// (include/Cellerator/compute/math/operation_core/operation_core.hh:214-237), with
// launch_bindings built from plain pointers handed over by the Python tests.
//
// `mutation` plants one defect in the request so a test can check the status the core or
// the backend reports, mirroring tests/math_core/operation_core_test.cc:120-270.
#include <cellerator_amd/cpmath/cpmath_backend.hh>

#include <chrono>
#include <cstdint>
#include <cstring>

namespace core = cellerator::compute::math::core;
namespace ex = cellerator::execution;
namespace cp = cellerator_amd::cpmath;

extern "C" {

typedef struct h_case {
    int32_t kind;  // 1 quantized CSR, 2 Blocked-ELL, 3 CP-BP
    int32_t mutation;
    const void *view;
    uint64_t view_bytes;
    uint32_t variant, rows, cols, out_cols, block_size, sparse_type, dense_type, reserved;
    uint64_t nnz;
    const void *values;
    uint64_t value_count, value_bytes;
    const void *scales, *offsets;
    const void *w;
    int64_t w_ld;
    void *y;
    int64_t y_ld;
    const void *w2;  // second launch of the same prepared operation (rebinding), if y2 != NULL
    void *y2;
    void *workspace;
    uint64_t workspace_bytes;
    void *stream;
    int32_t device, reserved2;
    // fused epilogue (multiply only): operation = spmm_operation(epilogue_kind, affine) when
    // fused != 0; bias (f32 [out_cols]) binds inputs[2] for the bias kinds; alpha / beta are
    // the affine effect's scalar bindings.
    uint32_t fused, epilogue_kind, affine, reserved3;
    const void *bias;
    float alpha, beta;
    // Physical preparations before the launch (cpmath_backend.hh): quantized CSR -- check the
    // column order (check_columns != 0) and interleave the plane's metadata into `pairs`
    // (non-NULL); Blocked-ELL -- pack W into `panel` (non-NULL) and use `groups` (non-NULL,
    // a cx_bell_groups). `repeats` runs the prepared operation that many times (0 -> 1).
    float *pairs;
    uint32_t check_columns, repeats;
    uint16_t *panel;
    const void *groups;
    // Quantized CSR through the execution-order candidate (exec_order != 0): 1 builds its
    // persistent state (prepare_quantized_csr_execution_order) before the launch, 2 does not
    // (the launch then runs the row-group kernel). head_genes goes into the declaration.
    // CP-BP: a non-NULL reduction_view (cx_cpbp_reduction_view) is validated once
    // (prepare_cpbp_state) before the launch.
    uint32_t exec_order, head_genes;
    const void *reduction_view;
    // with reduction_view: device u32 array (entry_rows_capacity) for the entry rows
    uint32_t *entry_rows;
    uint64_t entry_rows_capacity;
} h_case;

typedef struct h_result {
    int32_t prepare_status, status, binding, second_status;
    uint64_t kernel_low, kernel_high, workspace_bytes;
    uint32_t capability_flags, registered;
    int32_t state_status, reserved;
    char message[160];
    char engine[256];
    char dispatch[64];
    uint64_t persistent_bytes;  // execution-order state of the projection
    double launch_ms;           // repeats > 1: wall time per launch (stream synchronized around them)
} h_result;

int h_case_size(void) { return (int)sizeof(h_case); }
int h_result_size(void) { return (int)sizeof(h_result); }

}  // extern "C"

namespace {

enum mutation : int32_t {
    none = 0, stale_epoch = 1, structure_count = 2, short_workspace = 4, stale_generation = 5,
    bad_numeric = 6, wrong_projection_kind = 7, undeclared_projection = 8, swapped_axes = 9,
    output_aliases_input = 10, wrong_view_bytes = 11, values_in_view = 12, wrong_device = 15,
    wrong_dense_type = 16, wrong_output_shape = 17, tight_memory_policy = 18,
    retired_projection = 19, missing_scalars = 20, bias_numeric_mismatch = 21,
    f64_scalars = 22
};

ex::axis_identity axis(uint32_t base) {
    return {{base, 1u}, {base + 1u, 1u}, {base + 2u, 1u}, {base + 3u, 1u}};
}

ex::device_location device_at(int32_t ordinal) {
    ex::device_location l{};
    l.residency = ex::residency_kind::device;
    l.device_ordinal = ordinal;
    return l;
}

void note(h_result *r, const core::operation_status &s, bool prepare) {
    if (prepare) r->prepare_status = static_cast<int32_t>(s.code);
    else r->status = static_cast<int32_t>(s.code);
    r->binding = static_cast<int32_t>(s.binding);
    std::strncpy(r->message, s.message != nullptr ? s.message : "", sizeof(r->message) - 1u);
    std::strncpy(r->engine, cp::last_engine_error(), sizeof(r->engine) - 1u);
}

}  // namespace

extern "C" int h_run(const h_case *c, h_result *r) {
    std::memset(r, 0, sizeof(*r));
    r->prepare_status = r->status = r->second_status = -1;
    const ex::axis_identity cells = axis(100u), genes = axis(200u), outs = axis(300u);

    ex::relation_structure structure{};
    structure.identity = {5u, 1u};
    structure.epoch = {7u};
    structure.source_axis = cells;
    structure.destination_axis = genes;
    structure.projections = {1u, 1u};
    structure.logical_edge_count = c->nnz;

    const core::projection_kind kind = c->kind == 1 ? core::projection_kind::csr
        : c->kind == 2 ? core::projection_kind::blocked_ell
                       : core::projection_kind::native_row_masked;
    cp::projection_declaration d{};
    d.key = {{0x61u, 0x62u}, {9u, 1u}, kind, cp::physical_view_schema, c->variant};
    d.structure = structure;
    d.persistent_structure = {0x51u, 0x52u};
    d.output_axis = outs;
    d.rows = c->rows;
    d.cols = c->cols;
    d.output_columns = c->kind == 3 ? 0u : c->out_cols;
    d.block_size = c->block_size;
    d.head_genes = c->head_genes;
    core::operation_status s = cp::declare_projection(d);
    if (!s) { note(r, s, true); return 1; }

    core::candidate_registry registry{};
    const core::operation_candidate candidates[4] = {
        cp::quantized_csr_candidate(), cp::quantized_csr_execution_order_candidate(), cp::blocked_ell_candidate(),
        cp::cpbp_candidate()};
    for (const core::operation_candidate &candidate : candidates)
        if (core::register_candidate(&registry, candidate)) ++r->registered;
    const core::stable_id wanted = c->kind == 1
        ? (c->exec_order != 0u ? cp::quantized_csr_execution_order_candidate_id : cp::quantized_csr_candidate_id)
        : c->kind == 2 ? cp::blocked_ell_candidate_id : cp::cpbp_candidate_id;
    const core::operation_candidate *candidate = core::find_candidate(registry, wanted);
    if (candidate == nullptr) { cp::retire_projection(d.key.runtime); return 2; }
    r->capability_flags = candidate->capability_flags;

    const bool quantized = c->sparse_type == static_cast<uint32_t>(ex::numeric_type::u8);
    core::operation_problem problem{};
    problem.kind = candidate->operation;
    problem.operation = {0x71u, 0x72u};
    problem.input_count = 2u;
    if (c->fused != 0u) {
        problem.operation = cp::spmm_operation(c->epilogue_kind, c->affine != 0u);
        if (c->bias != nullptr) problem.input_count = 3u;
    }
    problem.output_count = 1u;
    problem.logical_work_items = c->rows;
    core::structure_set_key keys{};
    keys.count = 1u;
    keys.structures[0] = {d.persistent_structure, structure.identity, structure.epoch};
    core::projection_key projection = d.key;
    if (c->mutation == wrong_projection_kind)
        projection.kind = kind == core::projection_kind::csr ? core::projection_kind::blocked_ell
                                                             : core::projection_kind::csr;
    if (c->mutation == undeclared_projection) projection.runtime = {10u, 1u};
    core::numeric_policy numeric{};
    numeric.sparse_storage = static_cast<ex::numeric_type>(c->sparse_type);
    numeric.dense_storage = static_cast<ex::numeric_type>(c->dense_type);
    numeric.output_storage = ex::numeric_type::f32;
    numeric.multiply = ex::numeric_type::f32;
    numeric.accumulation = c->mutation == bad_numeric ? ex::numeric_type::f16 : ex::numeric_type::f32;
    numeric.scalar = ex::numeric_type::f32;
    numeric.bias = c->bias != nullptr ? ex::numeric_type::f32 : ex::numeric_type::invalid;
    if (c->mutation == bias_numeric_mismatch)
        numeric.bias = c->bias != nullptr ? ex::numeric_type::invalid : ex::numeric_type::f32;
    numeric.quantization = quantized ? core::quantization_granularity::module
                                     : core::quantization_granularity::none;
    core::prepare_policy policy{};
    policy.deterministic = true;
    policy.graph_capture_required = true;
    if (c->mutation == tight_memory_policy) policy.transient_memory_limit = 1024u;

    core::prepared_operation prepared{};
    s = core::prepare_candidate(*candidate, problem, keys, projection, numeric, policy, &prepared);
    note(r, s, true);
    if (!s) { cp::retire_projection(d.key.runtime); return 0; }
    r->kernel_low = prepared.kernel.low;
    r->kernel_high = prepared.kernel.high;
    r->workspace_bytes = prepared.binding_contract.workspace.minimum_bytes;
    if (c->mutation == retired_projection) cp::retire_projection(d.key.runtime);

    // ---- launch state ----
    ex::relation_structure bound = structure;
    if (c->mutation == stale_epoch) bound.epoch.value += 1u;
    ex::relation_structure extra = structure;
    extra.identity = {6u, 1u};
    const ex::relation_structure structures[2] = {bound, extra};

    ex::value_plane plane{};
    plane.structure = structure.identity;
    plane.structure_epoch_value = structure.epoch;
    plane.values = const_cast<void *>(c->values);
    plane.location = device_at(c->device);
    plane.numeric = {numeric.sparse_storage, ex::numeric_type::f32, ex::numeric_type::f32, 0u};
    if (quantized) {
        plane.quantization.kind = ex::quantization_kind::per_module;
        plane.quantization.scale_type = ex::numeric_type::f32;
        plane.quantization.offset_type = c->offsets != nullptr ? ex::numeric_type::f32
                                                               : ex::numeric_type::invalid;
        plane.quantization.scales = c->scales;
        plane.quantization.offsets = c->offsets;
        plane.quantization.group_count = c->cols;
    }
    plane.layout = c->kind == 1 ? ex::value_layout_kind::logical_edge_order
                                : ex::value_layout_kind::projection_local_order;
    plane.generation = {3u};
    plane.element_count = c->value_count;
    plane.value_bytes = c->value_bytes;
    const ex::value_binding values[1] = {
        {&plane, {c->mutation == stale_generation ? 4u : 3u}}};

    ex::biological_operand_view inputs[3]{};
    inputs[0].kind = ex::operand_kind::sparse_relation;
    ex::sparse_relation_view &rel = inputs[0].storage.relation;
    rel.source_axis = cells;
    rel.destination_axis = genes;
    rel.structure = structure.identity;
    rel.projection = d.key.runtime;
    rel.epoch = structure.epoch;
    rel.projection_data = c->view;
    rel.projection_bytes = c->mutation == wrong_view_bytes ? c->view_bytes + 8u : c->view_bytes;
    rel.logical_edge_count = c->nnz;
    rel.location = device_at(c->device);

    inputs[1].kind = ex::operand_kind::dense_tensor;
    ex::dense_tensor_view &w = inputs[1].storage.dense;
    w.data = const_cast<void *>(c->w);
    w.location = device_at(c->device);
    w.value_type = c->mutation == wrong_dense_type ? ex::numeric_type::f64
                                                   : static_cast<ex::numeric_type>(c->dense_type);
    ex::biological_operand_view outputs[1]{};
    outputs[0].kind = ex::operand_kind::dense_tensor;
    ex::dense_tensor_view &y = outputs[0].storage.dense;
    y.data = c->mutation == output_aliases_input ? const_cast<void *>(c->w) : c->y;
    y.location = device_at(c->device);
    y.value_type = ex::numeric_type::f32;
    if (c->kind == 3) {
        w.rank = 1u; w.axes[0] = genes; w.shape[0] = c->cols; w.stride[0] = 1;
        y.rank = 1u; y.axes[0] = cells; y.shape[0] = c->rows; y.stride[0] = 1;
    } else {
        w.rank = 2u; w.axes[0] = genes; w.axes[1] = outs;
        w.shape[0] = c->cols; w.shape[1] = c->out_cols; w.stride[0] = c->w_ld; w.stride[1] = 1;
        y.rank = 2u; y.axes[0] = cells; y.axes[1] = outs;
        y.shape[0] = c->rows; y.shape[1] = c->out_cols; y.stride[0] = c->y_ld; y.stride[1] = 1;
    }
    if (c->bias != nullptr) {
        inputs[2].kind = ex::operand_kind::dense_tensor;
        ex::dense_tensor_view &b = inputs[2].storage.dense;
        b.data = const_cast<void *>(c->bias);
        b.location = device_at(c->device);
        b.value_type = ex::numeric_type::f32;
        b.rank = 1u; b.axes[0] = outs; b.shape[0] = c->out_cols; b.stride[0] = 1;
    }
    if (c->mutation == swapped_axes) { w.axes[0] = outs; if (w.rank == 2u) w.axes[1] = genes; }
    if (c->mutation == wrong_output_shape) y.shape[0] += 1u;

    ex::launch_bindings launch{};
    launch.structures = structures;
    launch.structure_count = c->mutation == structure_count ? 2u : 1u;
    launch.inputs = inputs;
    launch.input_count = c->bias != nullptr ? 3u : 2u;
    if (c->affine != 0u && c->mutation != missing_scalars) {
        const bool wide = c->mutation == f64_scalars;
        const float scalars[2] = {c->alpha, c->beta};
        for (uint32_t i = 0; i < 2u; ++i) {
            ex::scalar_binding &b = launch.scalars.values[i];
            b.binding_id = i == 0u ? cp::alpha_binding : cp::beta_binding;
            b.type = wide ? ex::numeric_type::f64 : ex::numeric_type::f32;
            if (wide) {
                const double v = scalars[i];
                std::memcpy(&b.bits, &v, sizeof(v));
            } else {
                std::memcpy(&b.bits, &scalars[i], sizeof(float));
            }
        }
        launch.scalars.count = 2u;
    }
    launch.outputs = outputs;
    launch.output_count = 1u;
    launch.values = values;
    launch.value_count = 1u;
    launch.stream = {c->stream, c->device, 0u};
    launch.workspace.data = c->workspace;
    launch.workspace.bytes = c->mutation == short_workspace && c->workspace_bytes != 0u
        ? c->workspace_bytes - 1u : c->workspace_bytes;
    launch.workspace.location = device_at(c->mutation == wrong_device ? c->device + 1 : c->device);

    // A view with value pointers filled in is rejected: values travel in the value plane.
    alignas(16) unsigned char view_copy[256];
    if (c->mutation == values_in_view && c->view_bytes <= sizeof(view_copy)) {
        std::memcpy(view_copy, c->view, c->view_bytes);
        if (c->kind == 1) reinterpret_cast<cx_qcsr_matrix *>(view_copy)->packed_values =
            static_cast<const uint8_t *>(c->values);
        else if (c->kind == 2) reinterpret_cast<cx_bell_matrix *>(view_copy)->values = c->values;
        else reinterpret_cast<cx_cpbp_tiles *>(view_copy)->values = c->values;
        rel.projection_data = view_copy;
    }

    r->state_status = 0;
    if (c->kind == 1 && (c->check_columns != 0u || c->pairs != nullptr)) {
        const core::operation_status st = cp::prepare_quantized_csr_state(
            d.key.runtime, *static_cast<const cx_qcsr_matrix *>(c->view), &plane, c->pairs, c->stream);
        r->state_status = static_cast<int32_t>(st.code);
        if (!st) { note(r, st, false); cp::retire_projection(d.key.runtime); return 0; }
    }
    if (c->kind == 1 && c->exec_order == 1u) {
        const core::operation_status st = cp::prepare_quantized_csr_execution_order(
            d.key.runtime, *static_cast<const cx_qcsr_matrix *>(c->view), plane, c->stream);
        r->state_status = static_cast<int32_t>(st.code);
        r->persistent_bytes = cp::execution_order_persistent_bytes(d.key.runtime);
        if (!st) { note(r, st, false); cp::retire_projection(d.key.runtime); return 0; }
    }
    if (c->kind == 3 && c->reduction_view != nullptr) {
        const core::operation_status st = cp::prepare_cpbp_state(
            d.key.runtime, *static_cast<const cx_cpbp_reduction_view *>(c->reduction_view), c->entry_rows,
            c->entry_rows_capacity, c->stream);
        r->state_status = static_cast<int32_t>(st.code);
        if (!st) { note(r, st, false); cp::retire_projection(d.key.runtime); return 0; }
    }
    if (c->kind == 2 && (c->panel != nullptr || c->groups != nullptr)) {
        const core::operation_status st = cp::prepare_blocked_ell_state(
            d.key.runtime, *static_cast<const cx_bell_matrix *>(c->view),
            static_cast<const uint16_t *>(c->w), c->w_ld, c->panel,
            static_cast<const cx_bell_groups *>(c->groups), c->stream);
        r->state_status = static_cast<int32_t>(st.code);
        if (!st) { note(r, st, false); cp::retire_projection(d.key.runtime); return 0; }
    }

    // Several repeats are timed (stream synchronized before and after them); a single launch
    // is not, so it may run inside a HIP graph capture.
    const uint32_t repeats = c->repeats == 0u ? 1u : c->repeats;
    if (repeats > 1u) (void)cx_stream_synchronize(c->stream);
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t i = 0; i < repeats; ++i) {
        s = core::run_prepared_operation(prepared, launch);
        if (!s) break;
    }
    if (repeats > 1u) {
        (void)cx_stream_synchronize(c->stream);
        r->launch_ms =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / repeats;
    }
    note(r, s, false);
    std::strncpy(r->dispatch, cp::last_dispatch(), sizeof(r->dispatch) - 1u);
    if (s && c->y2 != nullptr) {
        // Rebinding without re-preparation: new W and Y pointers, same prepared record.
        w.data = const_cast<void *>(c->w2 != nullptr ? c->w2 : c->w);
        y.data = c->y2;
        const core::operation_status again = core::run_prepared_operation(prepared, launch);
        r->second_status = static_cast<int32_t>(again.code);
        std::strncpy(r->dispatch, cp::last_dispatch(), sizeof(r->dispatch) - 1u);
    }
    if (c->mutation != retired_projection) cp::retire_projection(d.key.runtime);
    return 0;
}
