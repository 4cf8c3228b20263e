// CP-Math operation-core backend: candidate records, prepare (freezes the binding contract
// from a declared projection) and run (checks the launch against the prepared projection,
// then calls the engine's C-ABI on the launch stream). The interface is described in
// cpmath_backend.hh.
#include "cpmath_backend.hh"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

namespace cellerator_amd::cpmath {
namespace {

using execution::i64;
using execution::numeric_type;
using execution::u32;
using execution::u64;
using code = core::operation_status_code;

constexpr u32 projection_capacity = 64u;
// The MFMA Blocked-ELL path packs W into the launch workspace: ceil(genes/32)*32 * N * 2
// bytes, at most this many (65,536 genes x 256 columns of bf16).
constexpr u64 mfma_panel_limit = 65536ull * 256ull * 2ull;

// Physical preparations of a quantized CSR projection (prepare_quantized_csr_state).
struct qcsr_prepared {
    bool sorted = false;                  // the structure below passed the column-order check
    const int32_t *row_ptr = nullptr;     // structure the check ran on
    const int32_t *col_idx = nullptr;
    float *pairs = nullptr;               // interleaved (scale, offset) of the plane below
    const void *scales = nullptr;
    const void *offsets = nullptr;
    u64 generation = 0u;
};

// The execution-order candidate's persistent state (prepare_quantized_csr_execution_order):
// the engine's prepared projection and what it was built from.
struct exec_prepared {
    cx_qcsr_exec_projection *projection = nullptr;
    const int32_t *row_ptr = nullptr;     // structure
    const int32_t *col_idx = nullptr;
    const void *values = nullptr;         // codes and metadata of the value plane
    const void *scales = nullptr;
    const void *offsets = nullptr;
    u64 generation = 0u;
    u64 persistent_bytes = 0u;
};

// Physical preparations of a Blocked-ELL projection (prepare_blocked_ell_state).
struct bell_prepared {
    const void *weights = nullptr;        // W the panel was packed from
    uint16_t *panel = nullptr;
    bool grouped = false;
    const uint32_t *block_col_idx = nullptr;  // structure the groups were planned on
    cx_bell_groups groups{};
};

// The validated reduction contract of a CP-BP projection (prepare_cpbp_state).
struct cpbp_prepared {
    bool validated = false;
    cx_cpbp_tiles tiles{};  // value pointer cleared: values travel in the plane
    const uint32_t *entry_rows = nullptr;  // cx_cpbp_entry_rows of `tiles` (caller-owned), or none
};

struct projection_state {
    bool live = false;
    projection_declaration declaration{};
    qcsr_prepared qcsr{};
    exec_prepared exec{};
    bell_prepared bell{};
    cpbp_prepared cpbp{};
    execution::operand_axis_contract inputs[3]{};  // sparse, dense, bias (epilogue only)
    execution::operand_axis_contract outputs[1]{};
    execution::output_axis_contract orders[2]{};
    execution::output_effect_contract effects[2]{};  // overwrite, affine_accumulate
    u32 order_count = 0u;
};

projection_state projections[projection_capacity];
std::mutex projections_mutex;
thread_local char engine_error[512] = "";
thread_local const char *dispatched = "";

constexpr core::operation_status fail(code c, const char *message) noexcept {
    return {c, execution::binding_validation_code::ok, message};
}

constexpr core::operation_status bad_launch(const char *message) noexcept {
    return {code::invalid_launch_bindings,
        execution::binding_validation_code::invalid_operand, message};
}

core::operation_status engine_failed(int rc) noexcept {
    const char *text = cx_last_error();
    std::strncpy(engine_error, text != nullptr ? text : "", sizeof(engine_error) - 1u);
    engine_error[sizeof(engine_error) - 1u] = '\0';
    return rc == CX_STATUS_HIP_ERROR
        ? fail(code::execution_failed, "engine kernel launch failed (see last_engine_error)")
        : fail(code::execution_failed, "engine rejected the launch (see last_engine_error)");
}

// ---- epilogue operations --------------------------------------------------------------

struct epilogue_request {
    std::uint32_t kind = CX_EPILOGUE_NONE;
    bool affine = false;
    bool bias = false;
};

// problem.operation -> epilogue; false for a malformed epilogue operation id.
bool parse_operation(const core::stable_id &operation, epilogue_request *out) noexcept {
    *out = epilogue_request{};
    if (operation.low != spmm_epilogue_family) return true;  // the plain product
    const u64 kind = operation.high & 0xffu;
    if ((operation.high & ~(0xffull | spmm_affine_flag)) != 0u || kind > CX_EPILOGUE_BIAS_GELU_TANH)
        return false;
    out->kind = static_cast<std::uint32_t>(kind);
    out->affine = (operation.high & spmm_affine_flag) != 0u;
    out->bias = kind == CX_EPILOGUE_BIAS || kind == CX_EPILOGUE_BIAS_RELU
        || kind == CX_EPILOGUE_BIAS_GELU_ERF || kind == CX_EPILOGUE_BIAS_GELU_TANH;
    return true;
}

bool is_epilogue_operation(const core::stable_id &operation) noexcept {
    return operation.low == spmm_epilogue_family;
}

// ---- numeric policies ----------------------------------------------------------------

bool common_numeric(const core::numeric_policy &n) noexcept {
    return n.output_storage == numeric_type::f32 && n.multiply == numeric_type::f32
        && n.accumulation == numeric_type::f32 && n.scalar == numeric_type::f32
        && n.rounding == core::rounding_policy::nearest_even
        && n.saturation == core::saturation_policy::none;
}

// Multiplies take an optional f32 bias (epilogue); the reduction takes none.
bool multiply_numeric(const core::numeric_policy &n) noexcept {
    return common_numeric(n) && (n.bias == numeric_type::invalid || n.bias == numeric_type::f32);
}

bool supports_quantized_csr(const core::numeric_policy &n) noexcept {
    if (!multiply_numeric(n)) return false;
    if (n.dense_storage != numeric_type::f16 && n.dense_storage != numeric_type::f32)
        return false;
    if (n.sparse_storage == numeric_type::u8)
        return n.quantization == core::quantization_granularity::module;
    return (n.sparse_storage == numeric_type::f16 || n.sparse_storage == numeric_type::f32)
        && n.quantization == core::quantization_granularity::none;
}

bool plain_storage(numeric_type t) noexcept {
    return t == numeric_type::bf16 || t == numeric_type::f16 || t == numeric_type::f32;
}

bool supports_blocked_ell(const core::numeric_policy &n) noexcept {
    return multiply_numeric(n) && plain_storage(n.sparse_storage)
        && plain_storage(n.dense_storage)
        && n.quantization == core::quantization_granularity::none;
}

bool supports_quantized_csr_execution_order(const core::numeric_policy &n) noexcept {
    return multiply_numeric(n) && n.dense_storage == numeric_type::f16
        && n.sparse_storage == numeric_type::u8 && n.quantization == core::quantization_granularity::module;
}

bool supports_cpbp(const core::numeric_policy &n) noexcept {
    return common_numeric(n) && n.bias == numeric_type::invalid
        && (n.sparse_storage == numeric_type::f16 || n.sparse_storage == numeric_type::f32)
        && n.dense_storage == numeric_type::f32
        && n.quantization == core::quantization_granularity::none;
}

std::uint32_t engine_dtype(numeric_type t) noexcept {
    switch (t) {
    case numeric_type::f16: return CELLERATOR_DTYPE_F16;
    case numeric_type::bf16: return CELLERATOR_DTYPE_BF16;
    case numeric_type::f32: return CELLERATOR_DTYPE_F32;
    default: return CELLERATOR_DTYPE_INVALID;
    }
}

// ---- launch checks --------------------------------------------------------------------

const projection_state *state_of(const core::prepared_operation &prepared) noexcept {
    if (prepared.persistent.data == nullptr
        || prepared.persistent.bytes != sizeof(projection_state))
        return nullptr;
    const auto *state = static_cast<const projection_state *>(prepared.persistent.data);
    if (!state->live
        || !execution::same_handle(state->declaration.key.runtime, prepared.projection.runtime))
        return nullptr;
    return state;
}

bool on_launch_device(const execution::device_location &where, const execution::launch_bindings &l) noexcept {
    return (where.residency == execution::residency_kind::device
               || where.residency == execution::residency_kind::managed)
        && where.device_ordinal == l.stream.device_ordinal;
}

// The sparse operand must carry the prepared projection and its structure, with the
// engine's physical view of `view_bytes` as projection data.
const void *physical_view(const projection_state &s, const execution::launch_bindings &l,
                          u64 view_bytes) noexcept {
    const execution::biological_operand_view &op = l.inputs[0];
    if (op.kind != execution::operand_kind::sparse_relation) return nullptr;
    const execution::sparse_relation_view &rel = op.storage.relation;
    if (!execution::same_handle(rel.projection, s.declaration.key.runtime)
        || !execution::same_handle(rel.structure, s.declaration.structure.identity)
        || rel.epoch.value != s.declaration.structure.epoch.value
        || rel.projection_bytes != view_bytes)
        return nullptr;
    return rel.projection_data;
}

const execution::value_plane *value_plane_of(const projection_state &s,
                                             const core::prepared_operation &p,
                                             const execution::launch_bindings &l) noexcept {
    if (l.value_count != 1u || l.values == nullptr || l.values[0].plane == nullptr) return nullptr;
    const execution::value_plane *plane = l.values[0].plane;
    if (!execution::same_handle(plane->structure, s.declaration.structure.identity)
        || plane->numeric.storage != p.numeric.sparse_storage
        || !on_launch_device(plane->location, l))
        return nullptr;
    return plane;
}

// Row-major matrix [rows x cols] (rank 2, unit inner stride) or vector [rows] (rank 1).
bool dense_shape(const execution::dense_tensor_view &v, numeric_type type, u32 rank, u64 rows,
                 u64 cols, const execution::launch_bindings &l) noexcept {
    if (v.value_type != type || v.rank != rank || v.shape[0] != rows || v.data == nullptr
        || !on_launch_device(v.location, l))
        return false;
    if (rank == 1u) return v.stride[0] == 1;
    return v.shape[1] == cols && v.stride[1] == 1 && v.stride[0] >= static_cast<i64>(cols);
}

// Launch-time epilogue of a prepared multiply: the bias operand (inputs[2]) and, for the
// affine effect, alpha / beta from the scalar bindings with Y itself as C.
bool scalar_value_of(const execution::launch_bindings &l, u32 id, float *value) noexcept {
    for (u32 i = 0u; i < l.scalars.count && i < execution::maximum_scalar_bindings; ++i) {
        const execution::scalar_binding &b = l.scalars.values[i];
        if (b.binding_id != id) continue;
        if (b.type == numeric_type::f32) {
            const std::uint32_t bits = static_cast<std::uint32_t>(b.bits);
            std::memcpy(value, &bits, sizeof(bits));
            return true;
        }
        if (b.type == numeric_type::f64) {
            double d;
            std::memcpy(&d, &b.bits, sizeof(d));
            *value = static_cast<float>(d);
            return true;
        }
        return false;
    }
    return false;
}

const char *bind_epilogue(const core::prepared_operation &p, const projection_declaration &d,
                          const execution::launch_bindings &l,
                          const execution::dense_tensor_view &y, cx_spmm_epilogue *ep) noexcept {
    epilogue_request e;
    if (!parse_operation(p.problem.operation, &e)) return "malformed epilogue operation";
    *ep = cx_spmm_epilogue{};
    ep->kind = e.kind;
    ep->alpha = 1.0f;
    if (e.bias) {
        if (l.input_count != 3u || l.inputs[2].kind != execution::operand_kind::dense_tensor
            || !dense_shape(l.inputs[2].storage.dense, numeric_type::f32, 1u, d.output_columns, 0u, l))
            return "bias must be a contiguous f32 [N] tensor";
        ep->bias = static_cast<const float *>(l.inputs[2].storage.dense.data);
    }
    if (e.affine) {
        if (!scalar_value_of(l, alpha_binding, &ep->alpha) || !scalar_value_of(l, beta_binding, &ep->beta))
            return "affine accumulation needs f32 or f64 alpha and beta scalars";
        ep->initial = static_cast<const float *>(y.data);
        ep->initial_ld = y.stride[0];
    }
    return nullptr;
}

// ---- run functions --------------------------------------------------------------------

// The launch operands of either quantized CSR candidate: the sparse view completed from the
// value plane (decode policy, codes, metadata, the prepared column order and pairs), W, Y and
// the epilogue. Returns a failure status, or ok.
struct qcsr_launch {
    cx_qcsr_matrix a{};
    const execution::value_plane *plane = nullptr;
    execution::dense_tensor_view w{};
    execution::dense_tensor_view y{};
    cx_spmm_epilogue ep{};
    bool sorted = false;
};

core::operation_status bind_quantized_csr(const projection_state &s, const core::prepared_operation &p,
                                          const execution::launch_bindings &l, qcsr_launch *out) noexcept {
    const projection_declaration &d = s.declaration;
    const void *view = physical_view(s, l, sizeof(cx_qcsr_matrix));
    if (view == nullptr) return bad_launch("sparse operand does not carry the prepared quantized CSR view");
    cx_qcsr_matrix &a = out->a;
    std::memcpy(&a, view, sizeof(a));
    if (a.rows != d.rows || a.cols != d.cols || a.bits != p.projection.variant
        || a.nnz != d.structure.logical_edge_count)
        return bad_launch("quantized CSR view differs from the declared projection");
    if (a.packed_values != nullptr || a.values != nullptr || a.column_scales != nullptr
        || a.column_offsets != nullptr || a.row_offsets != nullptr)
        return bad_launch("values and quantization metadata travel in the value plane");
    if (a.flags != 0u)
        return bad_launch("view flags are established by prepare_quantized_csr_state, not the caller");
    const execution::value_plane *plane = value_plane_of(s, p, l);
    if (plane == nullptr || plane->element_count != a.nnz)
        return bad_launch("one value plane of the structure with nnz elements is required");
    out->plane = plane;
    const execution::quantization_descriptor &q = plane->quantization;
    if (a.bits != 0u) {
        if (q.kind != execution::quantization_kind::per_module || q.group_count != a.cols
            || q.scale_type != numeric_type::f32
            || (q.offsets != nullptr && q.offset_type != numeric_type::f32))
            return bad_launch("quantized values need per-gene f32 scales (and offsets)");
        a.decode_policy = CX_DECODE_PER_GENE_AFFINE;
        a.packed_values = static_cast<const uint8_t *>(plane->values);
        a.column_scales = static_cast<const float *>(q.scales);
        a.column_offsets = static_cast<const float *>(q.offsets);
        const qcsr_prepared &pre = s.qcsr;
        if (pre.pairs != nullptr && pre.generation == plane->generation.value
            && pre.scales == q.scales && pre.offsets == q.offsets) {
            a.decode_policy = CX_DECODE_PER_GENE_AFFINE_PAIRS;
            a.column_scales = pre.pairs;
            a.column_offsets = nullptr;
        }
    } else {
        if (q.kind != execution::quantization_kind::none)
            return bad_launch("plain CSR values must not be quantized");
        a.values = plane->values;
        a.value_dtype = engine_dtype(plane->numeric.storage);
    }
    out->w = l.inputs[1].storage.dense;
    out->y = l.outputs[0].storage.dense;
    if (l.inputs[1].kind != execution::operand_kind::dense_tensor
        || !dense_shape(out->w, p.numeric.dense_storage, 2u, d.cols, d.output_columns, l))
        return bad_launch("W must be a row-major [genes x N] tensor of the dense storage type");
    if (!dense_shape(out->y, numeric_type::f32, 2u, d.rows, d.output_columns, l))
        return bad_launch("Y must be a row-major f32 [cells x N] tensor");
    if (const char *why = bind_epilogue(p, d, l, out->y, &out->ep)) return bad_launch(why);
    out->sorted = s.qcsr.sorted && s.qcsr.row_ptr == a.row_ptr && s.qcsr.col_idx == a.col_idx;
    if (out->sorted) a.flags = CX_QCSR_COLUMNS_SORTED;
    return {};
}

// The row-group (or row-wave) kernels on the bound CSR.
core::operation_status launch_row_group(const projection_state &s, qcsr_launch &q,
                                        const execution::launch_bindings &l) noexcept {
    const int rc = cx_qcsr_spmm_fwd_epilogue(&q.a, q.w.data, engine_dtype(q.w.value_type), q.w.stride[0],
                                             s.declaration.output_columns, static_cast<float *>(q.y.data),
                                             q.y.stride[0], &q.ep, l.stream.stream);
    return rc == CX_STATUS_SUCCESS ? core::operation_status{} : engine_failed(rc);
}

core::operation_status run_quantized_csr(const core::prepared_operation &p,
                                         const execution::launch_bindings &l) noexcept {
    const projection_state *s = state_of(p);
    if (s == nullptr) return fail(code::execution_failed, "prepared operation has no live projection state");
    qcsr_launch q;
    const core::operation_status bound = bind_quantized_csr(*s, p, l, &q);
    if (!bound) return bound;
    const core::operation_status st = launch_row_group(*s, q, l);
    if (!st) return st;
    const bool pairs = q.a.decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS;
    dispatched = q.a.bits == 0u ? "qcsr:plain"
        : pairs ? (q.sorted ? "qcsr:pairs+sorted" : "qcsr:pairs")
                : (q.sorted ? "qcsr:gene-affine+sorted" : "qcsr:gene-affine");
    return {};
}

// The execution-order candidate: the prepared projection when it was built from exactly the
// bound structure, codes and metadata, else the row-group kernel on the bound operands.
core::operation_status run_quantized_csr_execution_order(const core::prepared_operation &p,
                                                         const execution::launch_bindings &l) noexcept {
    const projection_state *s = state_of(p);
    if (s == nullptr) return fail(code::execution_failed, "prepared operation has no live projection state");
    qcsr_launch q;
    const core::operation_status bound = bind_quantized_csr(*s, p, l, &q);
    if (!bound) return bound;
    const exec_prepared &x = s->exec;
    const execution::quantization_descriptor &qd = q.plane->quantization;
    const bool current = x.projection != nullptr && x.row_ptr == q.a.row_ptr && x.col_idx == q.a.col_idx
        && x.values == q.plane->values && x.scales == qd.scales && x.offsets == qd.offsets
        && x.generation == q.plane->generation.value;
    const bool launchable = q.w.value_type == numeric_type::f16
        && (reinterpret_cast<std::uintptr_t>(q.y.data) & 15u) == 0u && (q.y.stride[0] * 4) % 16 == 0
        && q.y.data != q.w.data;
    if (!current || !launchable) {
        const core::operation_status st = launch_row_group(*s, q, l);
        if (st) dispatched = "qcsr:execution-order->row-group";
        return st;
    }
    const int rc = cx_qcsr_exec_spmm(x.projection, q.w.data, q.w.stride[0], s->declaration.output_columns,
                                     static_cast<float *>(q.y.data), q.y.stride[0], &q.ep, l.workspace.data,
                                     l.workspace.bytes, l.stream.stream);
    if (rc != CX_STATUS_SUCCESS) return engine_failed(rc);
    dispatched = "qcsr:execution-order";
    return {};
}

core::operation_status run_blocked_ell(const core::prepared_operation &p,
                                       const execution::launch_bindings &l) noexcept {
    const projection_state *s = state_of(p);
    if (s == nullptr) return fail(code::execution_failed, "prepared operation has no live projection state");
    const projection_declaration &d = s->declaration;
    const void *view = physical_view(*s, l, sizeof(cx_bell_matrix));
    if (view == nullptr) return bad_launch("sparse operand does not carry the prepared Blocked-ELL view");
    cx_bell_matrix a;
    std::memcpy(&a, view, sizeof(a));
    if (a.rows != d.rows || a.cols != d.cols || a.block_size != d.block_size || a.bits != 0u)
        return bad_launch("Blocked-ELL view differs from the declared projection");
    if (a.values != nullptr || a.packed_values != nullptr || a.column_scales != nullptr
        || a.column_offsets != nullptr || a.row_offsets != nullptr)
        return bad_launch("Blocked-ELL values travel in the value plane");
    if ((a.value_layout_flags != 0u && a.value_layout_flags != CX_BELL_BLOCK_MAJOR_VALUES) || a.reserved != 0u)
        return bad_launch("the projection-order value plane is row-major [rows x ell_cols] or block-major");
    const execution::value_plane *plane = value_plane_of(*s, p, l);
    if (plane == nullptr || plane->layout != execution::value_layout_kind::projection_local_order
        || plane->quantization.kind != execution::quantization_kind::none
        || plane->element_count != static_cast<u64>(a.rows) * a.ell_cols)
        return bad_launch("one projection-order value plane of rows x ell_cols values is required");
    a.values = plane->values;
    a.value_dtype = engine_dtype(plane->numeric.storage);
    const execution::dense_tensor_view &w = l.inputs[1].storage.dense;
    const execution::dense_tensor_view &y = l.outputs[0].storage.dense;
    if (l.inputs[1].kind != execution::operand_kind::dense_tensor
        || !dense_shape(w, p.numeric.dense_storage, 2u, d.cols, d.output_columns, l))
        return bad_launch("W must be a row-major [genes x N] tensor of the dense storage type");
    if (!dense_shape(y, numeric_type::f32, 2u, d.rows, d.output_columns, l))
        return bad_launch("Y must be a row-major f32 [cells x N] tensor");
    cx_spmm_epilogue ep;
    if (const char *why = bind_epilogue(p, d, l, y, &ep)) return bad_launch(why);
    int rc;
    if (core::same_stable_id(p.kernel, blocked_ell_mfma_kernel_id)) {
        const bell_prepared &pre = s->bell;
        const bool prepacked = pre.panel != nullptr && pre.weights == w.data;
        const uint16_t *panel = pre.panel;
        rc = CX_STATUS_SUCCESS;
        if (!prepacked) {
            auto *scratch = static_cast<uint16_t *>(l.workspace.data);
            rc = cx_bell_pack_rhs(static_cast<const uint16_t *>(w.data), w.stride[0], d.cols,
                                  d.output_columns, scratch, l.stream.stream);
            panel = scratch;
        }
        const bool grouped = pre.grouped && pre.block_col_idx == a.block_col_idx;
        if (rc == CX_STATUS_SUCCESS)
            rc = grouped
                ? cx_bell_spmm_fwd_grouped_epilogue(&a, panel, &pre.groups, d.output_columns,
                                                    static_cast<float *>(y.data), y.stride[0], &ep,
                                                    l.stream.stream)
                : cx_bell_spmm_fwd_packed_epilogue(&a, panel, d.output_columns,
                                                   static_cast<float *>(y.data), y.stride[0], &ep,
                                                   l.stream.stream);
        const bool block_major = a.value_layout_flags == CX_BELL_BLOCK_MAJOR_VALUES;
        dispatched = grouped ? (prepacked ? (block_major ? "bell:grouped+panel+block-major" : "bell:grouped+panel")
                                          : (block_major ? "bell:grouped+repack+block-major" : "bell:grouped+repack"))
                             : (prepacked ? (block_major ? "bell:mfma+panel+block-major" : "bell:mfma+panel")
                                          : (block_major ? "bell:mfma+repack+block-major" : "bell:mfma+repack"));
    } else {
        rc = cx_bell_spmm_fwd_epilogue(&a, w.data, engine_dtype(w.value_type), w.stride[0],
                                       d.output_columns, static_cast<float *>(y.data),
                                       y.stride[0], &ep, l.stream.stream);
        dispatched = "bell:generic";
    }
    return rc == CX_STATUS_SUCCESS ? core::operation_status{} : engine_failed(rc);
}

core::operation_status run_cpbp(const core::prepared_operation &p,
                                const execution::launch_bindings &l) noexcept {
    const projection_state *s = state_of(p);
    if (s == nullptr) return fail(code::execution_failed, "prepared operation has no live projection state");
    const projection_declaration &d = s->declaration;
    // The engine's tile view, or the reference's native tile view (its math projection of
    // the same partition, native_tile_view.hh:45-54), which aliases the compact values.
    cx_cpbp_tiles t;
    bool native = false;
    const void *view = physical_view(*s, l, sizeof(cx_cpbp_tiles));
    if (view != nullptr) {
        std::memcpy(&t, view, sizeof(t));
        if (t.values != nullptr) return bad_launch("CP-BP values travel in the value plane");
    } else if ((view = physical_view(*s, l, sizeof(cx_native_tile_view))) != nullptr) {
        cx_native_tile_view nv;
        std::memcpy(&nv, view, sizeof(nv));
        if (nv.packed_value_offsets == nullptr || cx_cpbp_tiles_from_native_view(&nv, &t) != CX_STATUS_SUCCESS)
            return bad_launch("sparse operand's native tile view is not a built v1 view");
        native = true;
    } else {
        return bad_launch("sparse operand does not carry the prepared CP-BP tile view");
    }
    if (t.row_count != d.rows || t.feature_count != d.cols
        || t.nnz_count != d.structure.logical_edge_count)
        return bad_launch("CP-BP tile view differs from the declared projection");
    const void *aliased = t.values;
    const bool checked = s->cpbp.validated;
    if (checked) {
        cx_cpbp_tiles bound = t;  // the plane supplies values and their type
        bound.values = nullptr;
        bound.value_dtype = 0u;
        if (std::memcmp(&bound, &s->cpbp.tiles, sizeof(bound)) != 0)
            return bad_launch("CP-BP tile view differs from the reduction view validated by prepare_cpbp_state");
    }
    const execution::value_plane *plane = value_plane_of(*s, p, l);
    if (plane == nullptr || plane->layout != execution::value_layout_kind::projection_local_order
        || plane->quantization.kind != execution::quantization_kind::none
        || plane->element_count != t.nnz_count)
        return bad_launch("one projection-order value plane of nnz values is required");
    if (native && aliased != nullptr && aliased != plane->values)
        return bad_launch("the native tile view's values are not the bound value plane");
    t.values = plane->values;
    t.value_dtype = engine_dtype(plane->numeric.storage);
    const execution::dense_tensor_view &w = l.inputs[1].storage.dense;
    const execution::dense_tensor_view &y = l.outputs[0].storage.dense;
    if (l.inputs[1].kind != execution::operand_kind::dense_tensor
        || !dense_shape(w, numeric_type::f32, 1u, d.cols, 0u, l))
        return bad_launch("feature weights must be a contiguous f32 [genes] tensor");
    if (!dense_shape(y, numeric_type::f32, 1u, d.rows, 0u, l))
        return bad_launch("row values must be a contiguous f32 [cells] tensor");
    // with the validated structure's entry rows, each entry's row and block start are read
    // instead of looked up from its descriptor (bitwise the same sums)
    const bool rows = checked && s->cpbp.entry_rows != nullptr;
    const int rc = rows ? cx_cpbp_reduce_rows(&t, s->cpbp.entry_rows, static_cast<const float *>(w.data), d.cols,
                                              static_cast<float *>(y.data), d.rows, l.stream.stream)
                        : cx_cpbp_reduce(&t, static_cast<const float *>(w.data), d.cols,
                                         static_cast<float *>(y.data), d.rows, l.stream.stream);
    if (rc != CX_STATUS_SUCCESS) return engine_failed(rc);
    dispatched = native ? (rows ? "cpbp:native-tile+checked+entry-rows"
                                : checked ? "cpbp:native-tile+checked" : "cpbp:native-tile")
                        : (rows ? "cpbp:checked+entry-rows" : checked ? "cpbp:checked" : "cpbp:unchecked");
    return {};
}

// ---- prepare --------------------------------------------------------------------------

projection_state *find_live(execution::projection_handle handle) noexcept {
    for (projection_state &s : projections)
        if (s.live && execution::same_handle(s.declaration.key.runtime, handle)) return &s;
    return nullptr;
}

// Matrix-core head width of the execution-order candidate.
std::uint32_t head_genes_of(const projection_declaration &d) noexcept {
    return d.head_genes != 0u ? d.head_genes : 2048u;
}

u64 mfma_panel_bytes(const projection_declaration &d) noexcept {
    return (static_cast<u64>(d.cols) + 31u) / 32u * 32u * d.output_columns * 2u;
}

bool mfma_eligible(const projection_declaration &d, const core::numeric_policy &n) noexcept {
    return n.sparse_storage == numeric_type::bf16 && n.dense_storage == numeric_type::bf16
        && d.block_size == 32u
        && (d.output_columns == 64u || d.output_columns == 128u || d.output_columns == 256u)
        && mfma_panel_bytes(d) <= mfma_panel_limit;
}

core::operation_status prepare(
    const core::operation_candidate &candidate,
    const core::operation_problem &problem,
    const core::structure_set_key &structures,
    const core::projection_key &projection,
    const core::numeric_policy &numeric,
    const core::prepare_policy &policy,
    core::prepared_operation *prepared) noexcept {
    if (prepared == nullptr) return fail(code::invalid_argument, "prepare needs an output record");
    std::lock_guard<std::mutex> lock(projections_mutex);
    projection_state *state = find_live(projection.runtime);
    if (state == nullptr)
        return fail(code::unsupported_projection, "projection was not declared to the engine backend");
    const projection_declaration &d = state->declaration;
    if (!execution::same_identity(d.key.persistent, projection.persistent)
        || d.key.kind != projection.kind || d.key.schema_version != projection.schema_version
        || d.key.variant != projection.variant || candidate.projection != projection.kind)
        return fail(code::unsupported_projection, "projection key differs from its declaration");
    if (structures.count != 1u
        || !execution::same_handle(structures.structures[0].runtime, d.structure.identity)
        || structures.structures[0].epoch.value != d.structure.epoch.value
        || !execution::same_identity(structures.structures[0].persistent, d.persistent_structure))
        return {code::stale_structure, execution::binding_validation_code::stale_structure,
            "structure key differs from the declared projection's structure"};
    epilogue_request epilogue;
    if (!parse_operation(problem.operation, &epilogue))
        return fail(code::unsupported_problem, "unknown epilogue in the operation identity");
    const bool reduce = candidate.operation == core::operation_kind::weighted_relation_reduce;
    if (reduce && is_epilogue_operation(problem.operation))
        return fail(code::unsupported_problem, "the row reduction has no epilogue");
    if (epilogue.bias != (numeric.bias == numeric_type::f32))
        return fail(code::unsupported_numeric_policy,
            "a bias epilogue needs numeric bias f32, and only a bias epilogue may declare one");
    const u32 input_count = epilogue.bias ? 3u : 2u;
    if (problem.input_count != input_count || problem.output_count != 1u)
        return fail(code::unsupported_problem,
            "operation takes one sparse and one dense input (plus the bias) and one output");
    if (projection.kind == core::projection_kind::csr
        && (projection.variant != 0u) != (numeric.sparse_storage == numeric_type::u8))
        return fail(code::unsupported_numeric_policy,
            "code width in the projection variant disagrees with the sparse storage type");

    core::stable_id kernel = candidate.identity;
    core::run_function run = run_quantized_csr;
    u64 workspace = 0u;
    if (reduce) {
        run = run_cpbp;
    } else if (core::same_stable_id(candidate.identity, quantized_csr_execution_order_candidate_id)) {
        if (projection.variant == 0u || numeric.dense_storage != numeric_type::f16
            || d.output_columns % 64u != 0u || d.output_columns > 256u)
            return fail(code::unsupported_numeric_policy,
                "the execution-order candidate needs quantized codes, f16 W and N of 64, 128, 192 or 256");
        if (cx_qcsr_exec_workspace_for(d.rows, d.cols, head_genes_of(d), d.output_columns, &workspace)
            != CX_STATUS_SUCCESS)
            return fail(code::unsupported_problem, "execution-order workspace is not defined for this shape");
        if (policy.persistent_memory_limit != 0u && state->exec.persistent_bytes > policy.persistent_memory_limit)
            return fail(code::capability_rejected, "candidate exceeds memory policy");
        run = run_quantized_csr_execution_order;
    } else if (projection.kind == core::projection_kind::blocked_ell) {
        const bool mfma = mfma_eligible(d, numeric);
        kernel = mfma ? blocked_ell_mfma_kernel_id : blocked_ell_generic_kernel_id;
        workspace = mfma ? mfma_panel_bytes(d) : 0u;
        run = run_blocked_ell;
    }
    if (policy.transient_memory_limit != 0u && workspace > policy.transient_memory_limit)
        return fail(code::capability_rejected, "candidate exceeds memory policy");

    *prepared = core::prepared_operation{};
    prepared->problem = problem;
    prepared->structures = structures;
    prepared->projection = projection;
    prepared->numeric = numeric;
    prepared->kernel = kernel;
    prepared->backend = core::backend_kind::native_direct;
    prepared->capability_flags = candidate.capability_flags;
    prepared->persistent = {state, sizeof(*state)};
    prepared->binding_contract.structures[0] = {d.structure.identity, d.structure.epoch};
    prepared->binding_contract.inputs = state->inputs;
    prepared->binding_contract.outputs = state->outputs;
    prepared->binding_contract.output_orders = state->orders;
    prepared->binding_contract.output_effects = &state->effects[epilogue.affine ? 1 : 0];
    prepared->binding_contract.input_count = input_count;
    prepared->binding_contract.output_count = 1u;
    prepared->binding_contract.output_order_count = state->order_count;
    prepared->binding_contract.structure_count = 1u;
    prepared->binding_contract.output_effect_count = 1u;
    prepared->binding_contract.workspace = {workspace, 256u, 0u};
    prepared->run = run;
    return {};
}

core::operation_candidate candidate(core::stable_id id, const char *name,
                                    core::operation_kind operation,
                                    core::projection_kind projection,
                                    core::numeric_support_function supports,
                                    u64 transient_bytes, std::uint32_t extra_flags = 0u) noexcept {
    core::operation_candidate c{};
    c.identity = id;
    c.name = name;
    c.operation = operation;
    c.projection = projection;
    c.backend = core::backend_kind::native_direct;
    // Fixed per-row / per-tile summation order, and launches that neither allocate nor
    // synchronize.
    c.capability_flags = core::candidate_deterministic | core::candidate_graph_capture | extra_flags;
    // Device-resident state beyond the caller's operands depends on the projection: the
    // execution-order candidate checks its prepared bytes against the policy in prepare.
    c.persistent_bytes = 0u;
    c.transient_bytes = transient_bytes;
    c.supports_numeric = supports;
    c.prepare = prepare;
    return c;
}

} // namespace

core::operation_status declare_projection(const projection_declaration &d) noexcept {
    const core::projection_key &k = d.key;
    if (!execution::valid_identity(k.persistent) || !execution::valid_handle(k.runtime)
        || k.schema_version != physical_view_schema)
        return fail(code::invalid_argument, "projection key is incomplete or of another schema");
    const bool multiply = k.kind == core::projection_kind::csr
        || k.kind == core::projection_kind::blocked_ell;
    if (!multiply && k.kind != core::projection_kind::native_row_masked)
        return fail(code::unsupported_projection, "engine backend serves csr, blocked_ell and native_row_masked");
    if (execution::validate_relation_structure(d.structure) != execution::lifetime_validation_code::ok
        || !execution::valid_identity(d.persistent_structure))
        return fail(code::stale_structure, "relation structure is invalid");
    if (d.rows == 0u || d.cols == 0u)
        return fail(code::invalid_argument, "projection needs rows and genes");
    if (multiply && (d.output_columns == 0u || !execution::valid_axis_identity(d.output_axis)))
        return fail(code::invalid_argument, "multiply projection needs an output axis and N");
    if (!multiply && d.output_columns != 0u)
        return fail(code::invalid_argument, "the row reduction has no output columns");
    if (k.kind == core::projection_kind::csr && k.variant != 0u && k.variant != 1u
        && k.variant != 2u && k.variant != 4u && k.variant != 8u)
        return fail(code::unsupported_projection, "quantized CSR code width must be 1, 2, 4 or 8");
    if (k.kind == core::projection_kind::blocked_ell && d.block_size == 0u)
        return fail(code::invalid_argument, "Blocked-ELL projection needs its block size");

    std::lock_guard<std::mutex> lock(projections_mutex);
    if (find_live(k.runtime) != nullptr)
        return fail(code::duplicate_candidate, "projection is already declared");
    projection_state *slot = nullptr;
    for (projection_state &s : projections)
        if (!s.live) { slot = &s; break; }
    if (slot == nullptr) return fail(code::registry_full, "projection table is full");

    *slot = projection_state{};
    slot->declaration = d;
    const execution::axis_identity cells = d.structure.source_axis;
    const execution::axis_identity genes = d.structure.destination_axis;
    slot->inputs[0].kind = execution::operand_kind::sparse_relation;
    slot->inputs[0].rank = 2u;
    slot->inputs[0].axes[0] = cells;
    slot->inputs[0].axes[1] = genes;
    slot->inputs[1].kind = execution::operand_kind::dense_tensor;
    slot->outputs[0].kind = execution::operand_kind::dense_tensor;
    slot->orders[0].input_axis = cells;
    slot->orders[0].output_axis = cells;
    slot->orders[0].transition = execution::order_transition_kind::preserve;
    slot->orders[0].axis_index = 0u;
    if (multiply) {
        slot->inputs[1].rank = 2u;
        slot->inputs[1].axes[0] = genes;
        slot->inputs[1].axes[1] = d.output_axis;
        slot->inputs[2].kind = execution::operand_kind::dense_tensor;
        slot->inputs[2].rank = 1u;
        slot->inputs[2].axes[0] = d.output_axis;
        slot->outputs[0].rank = 2u;
        slot->outputs[0].axes[0] = cells;
        slot->outputs[0].axes[1] = d.output_axis;
        slot->orders[1].input_axis = d.output_axis;
        slot->orders[1].output_axis = d.output_axis;
        slot->orders[1].transition = execution::order_transition_kind::preserve;
        slot->orders[1].axis_index = 1u;
        slot->order_count = 2u;
    } else {
        slot->inputs[1].rank = 1u;
        slot->inputs[1].axes[0] = genes;
        slot->outputs[0].rank = 1u;
        slot->outputs[0].axes[0] = cells;
        slot->order_count = 1u;
    }
    slot->effects[0] = {execution::output_update_kind::overwrite, false, false, 0u,
        execution::invalid_scalar_binding_id, execution::invalid_scalar_binding_id};
    slot->effects[1] = {execution::output_update_kind::affine_accumulate, true, false, 0u,
        alpha_binding, beta_binding};
    slot->live = true;
    return {};
}

core::operation_status retire_projection(execution::projection_handle projection) noexcept {
    std::lock_guard<std::mutex> lock(projections_mutex);
    projection_state *s = find_live(projection);
    if (s == nullptr) return fail(code::invalid_argument, "projection is not declared");
    if (s->exec.projection != nullptr) (void)cx_qcsr_exec_destroy(s->exec.projection);
    s->exec = exec_prepared{};
    s->live = false;
    return {};
}

core::operation_candidate quantized_csr_candidate() noexcept {
    return candidate(quantized_csr_candidate_id, "cellerator-amd-quantized-csr-spmm",
        core::operation_kind::sparse_dense_multiply, core::projection_kind::csr,
        supports_quantized_csr, 0u);
}

core::operation_candidate quantized_csr_execution_order_candidate() noexcept {
    return candidate(quantized_csr_execution_order_candidate_id, "cellerator-amd-quantized-csr-execution-order",
        core::operation_kind::sparse_dense_multiply, core::projection_kind::csr,
        supports_quantized_csr_execution_order, 0u, core::candidate_persistent_preprocessing);
}

core::operation_candidate blocked_ell_candidate() noexcept {
    return candidate(blocked_ell_candidate_id, "cellerator-amd-blocked-ell-spmm",
        core::operation_kind::sparse_dense_multiply, core::projection_kind::blocked_ell,
        supports_blocked_ell, mfma_panel_limit);
}

core::operation_candidate cpbp_candidate() noexcept {
    return candidate(cpbp_candidate_id, "cellerator-amd-cpbp-row-reduction",
        core::operation_kind::weighted_relation_reduce, core::projection_kind::native_row_masked,
        supports_cpbp, 0u);
}

core::operation_status prepare_quantized_csr_state(execution::projection_handle projection,
                                                   const cx_qcsr_matrix &structure,
                                                   const execution::value_plane *plane,
                                                   float *pairs, void *stream) noexcept {
    std::lock_guard<std::mutex> lock(projections_mutex);
    projection_state *s = find_live(projection);
    if (s == nullptr) return fail(code::invalid_argument, "projection is not declared");
    const projection_declaration &d = s->declaration;
    if (d.key.kind != core::projection_kind::csr)
        return fail(code::unsupported_projection, "not a quantized CSR projection");
    if (structure.rows != d.rows || structure.cols != d.cols
        || structure.nnz != d.structure.logical_edge_count || structure.row_ptr == nullptr
        || (structure.nnz != 0u && structure.col_idx == nullptr))
        return fail(code::invalid_argument, "structure differs from the declared projection");
    qcsr_prepared pre{};
    if (pairs != nullptr) {
        if (plane == nullptr || d.key.variant == 0u
            || plane->quantization.kind != execution::quantization_kind::per_module
            || plane->quantization.scale_type != numeric_type::f32
            || plane->quantization.group_count != d.cols
            || (plane->quantization.offsets != nullptr
                && plane->quantization.offset_type != numeric_type::f32)
            || !execution::same_handle(plane->structure, d.structure.identity))
            return fail(code::invalid_argument, "pairs need the projection's per-gene f32 quantization plane");
        int rc = cx_qcsr_pack_gene_affine(static_cast<const float *>(plane->quantization.scales),
                                          static_cast<const float *>(plane->quantization.offsets),
                                          d.cols, pairs, stream);
        if (rc != CX_STATUS_SUCCESS) return engine_failed(rc);
        pre.pairs = pairs;
        pre.scales = plane->quantization.scales;
        pre.offsets = plane->quantization.offsets;
        pre.generation = plane->generation.value;
    }
    uint32_t host_flag = 0u;
    const int rc = cx_qcsr_check_columns_sync(&structure, &host_flag, stream);
    if (rc != CX_STATUS_SUCCESS) return engine_failed(rc);
    pre.sorted = (host_flag & CX_QCSR_COLUMNS_SORTED) != 0u;
    pre.row_ptr = structure.row_ptr;
    pre.col_idx = structure.col_idx;
    s->qcsr = pre;
    return {};
}

core::operation_status prepare_quantized_csr_execution_order(execution::projection_handle projection,
                                                             const cx_qcsr_matrix &structure,
                                                             const execution::value_plane &plane,
                                                             void *stream) noexcept {
    std::lock_guard<std::mutex> lock(projections_mutex);
    projection_state *s = find_live(projection);
    if (s == nullptr) return fail(code::invalid_argument, "projection is not declared");
    const projection_declaration &d = s->declaration;
    if (d.key.kind != core::projection_kind::csr || d.key.variant == 0u)
        return fail(code::unsupported_projection, "not a quantized CSR projection");
    if (structure.rows != d.rows || structure.cols != d.cols || structure.bits != d.key.variant
        || structure.nnz != d.structure.logical_edge_count || structure.row_ptr == nullptr
        || structure.packed_row_ptr == nullptr || (structure.nnz != 0u && structure.col_idx == nullptr))
        return fail(code::invalid_argument, "structure differs from the declared projection");
    const execution::quantization_descriptor &q = plane.quantization;
    if (!execution::same_handle(plane.structure, d.structure.identity)
        || q.kind != execution::quantization_kind::per_module || q.group_count != d.cols
        || q.scale_type != numeric_type::f32 || (q.offsets != nullptr && q.offset_type != numeric_type::f32)
        || plane.values == nullptr || plane.element_count != structure.nnz)
        return fail(code::invalid_argument, "the execution order needs the projection's codes with per-gene f32 metadata");
    cx_qcsr_matrix a = structure;
    a.decode_policy = CX_DECODE_PER_GENE_AFFINE;
    a.packed_values = static_cast<const uint8_t *>(plane.values);
    a.column_scales = static_cast<const float *>(q.scales);
    a.column_offsets = static_cast<const float *>(q.offsets);
    a.row_offsets = nullptr;
    a.values = nullptr;
    a.flags = 0u;
    if (s->exec.projection != nullptr) (void)cx_qcsr_exec_destroy(s->exec.projection);
    s->exec = exec_prepared{};
    cx_qcsr_exec_projection *x = nullptr;
    const int rc = cx_qcsr_exec_prepare(&a, head_genes_of(d), &x, stream);
    if (rc != CX_STATUS_SUCCESS) {
        const core::operation_status st = engine_failed(rc);
        return {code::preparation_failed, st.binding, "execution-order preparation failed (see last_engine_error)"};
    }
    cx_qcsr_exec_info info{};
    (void)cx_qcsr_exec_query(x, &info);
    exec_prepared e{};
    e.projection = x;
    e.row_ptr = structure.row_ptr;
    e.col_idx = structure.col_idx;
    e.values = plane.values;
    e.scales = q.scales;
    e.offsets = q.offsets;
    e.generation = plane.generation.value;
    e.persistent_bytes = info.persistent_bytes;
    s->exec = e;
    return {};
}

std::uint64_t execution_order_persistent_bytes(execution::projection_handle projection) noexcept {
    std::lock_guard<std::mutex> lock(projections_mutex);
    const projection_state *s = find_live(projection);
    return s != nullptr ? s->exec.persistent_bytes : 0u;
}

core::operation_status prepare_cpbp_state(execution::projection_handle projection,
                                          const cx_cpbp_reduction_view &view, uint32_t *entry_rows,
                                          uint64_t entry_rows_capacity, void *stream) noexcept {
    std::lock_guard<std::mutex> lock(projections_mutex);
    projection_state *s = find_live(projection);
    if (s == nullptr) return fail(code::invalid_argument, "projection is not declared");
    const projection_declaration &d = s->declaration;
    if (d.key.kind != core::projection_kind::native_row_masked)
        return fail(code::unsupported_projection, "not a CP-BP projection");
    if (view.tiles.row_count != d.rows || view.tiles.feature_count != d.cols
        || view.tiles.nnz_count != d.structure.logical_edge_count)
        return fail(code::invalid_argument, "reduction view differs from the declared projection");
    const int rc = cx_cpbp_reduction_validate(&view);
    if (rc != CX_STATUS_SUCCESS) {
        const core::operation_status st = engine_failed(rc);
        return {code::preparation_failed, st.binding, "reduction contract rejected (see last_engine_error)"};
    }
    if (entry_rows != nullptr) {
        const int er = cx_cpbp_entry_rows(&view.tiles, entry_rows, entry_rows_capacity, stream);
        if (er != CX_STATUS_SUCCESS) {
            const core::operation_status st = engine_failed(er);
            return {code::preparation_failed, st.binding, "entry rows rejected (see last_engine_error)"};
        }
    }
    s->cpbp.validated = true;
    s->cpbp.tiles = view.tiles;
    s->cpbp.tiles.values = nullptr;
    s->cpbp.tiles.value_dtype = 0u;
    s->cpbp.entry_rows = entry_rows;
    return {};
}

core::operation_status prepare_blocked_ell_state(execution::projection_handle projection,
                                                 const cx_bell_matrix &structure,
                                                 const uint16_t *weights, int64_t weights_ld,
                                                 uint16_t *panel, const cx_bell_groups *groups,
                                                 void *stream) noexcept {
    std::lock_guard<std::mutex> lock(projections_mutex);
    projection_state *s = find_live(projection);
    if (s == nullptr) return fail(code::invalid_argument, "projection is not declared");
    const projection_declaration &d = s->declaration;
    if (d.key.kind != core::projection_kind::blocked_ell)
        return fail(code::unsupported_projection, "not a Blocked-ELL projection");
    if (structure.rows != d.rows || structure.cols != d.cols || structure.block_size != d.block_size
        || structure.block_col_idx == nullptr)
        return fail(code::invalid_argument, "structure differs from the declared projection");
    bell_prepared pre{};
    if (panel != nullptr) {
        if (weights == nullptr) return fail(code::invalid_argument, "the panel is packed from weights");
        int rc = cx_bell_pack_rhs(weights, weights_ld, d.cols, d.output_columns, panel, stream);
        if (rc == CX_STATUS_SUCCESS) rc = cx_stream_synchronize(stream);
        if (rc != CX_STATUS_SUCCESS) return engine_failed(rc);
        pre.weights = weights;
        pre.panel = panel;
    }
    if (groups != nullptr) {
        pre.grouped = true;
        pre.groups = *groups;
        pre.block_col_idx = structure.block_col_idx;
    }
    s->bell = pre;
    return {};
}

const char *last_dispatch() noexcept { return dispatched; }

namespace {

// Peaks of one MI355X and the fraction of them each kernel family reaches on the
// benchmark configurations (measured with bench.py on one MI355X: the quantized CSR
// row-group kernel at 35% of the non-packed fp32 VALU peak (C3: 6.99 ms for 2*nnz*N flops);
// the execution-order path at 74% of it (C3: 3.31 ms, head on the matrix cores plus the
// tail stream) after a preparation of about 0.028 ns per stored entry (C3: 41 ms); the
// Blocked-ELL grouped matrix-core kernel on its launch schedule at about 47% of HBM (C4:
// 0.52 ms); the CP-BP reduction at about 48% of HBM from the descriptors (C5: 1.2 ms), 55%
// with prepared entry rows).
constexpr double kHbmBytesPerNs = 8000.0;         // 8 TB/s
constexpr double kValuFlopsPerNs = 78600.0;        // fp32, non-packed
constexpr double kMfmaFlopsPerNs = 2500000.0;      // bf16 dense
constexpr double kQcsrEfficiency = 0.35, kBellEfficiency = 0.47, kCpbpEfficiency = 0.48;
constexpr double kQcsrExecEfficiency = 0.74;
constexpr double kQcsrExecPrepareNsPerEntry = 0.028;
constexpr double kLaunchNs = 4000.0;               // launch and synchronization overhead

double align256d(double bytes) { return std::ceil(bytes / 256.0) * 256.0; }

bool finite_shape(const workload_shape &w) { return w.rows != 0u && w.cols != 0u; }

} // namespace

bool analytical_costs(core::stable_id candidate, const workload_shape &w,
                      cellerator::planner::phase_costs *out) noexcept {
    if (out == nullptr || !finite_shape(w)) return false;
    cellerator::planner::phase_costs p{};
    p.host_preparation_ns = 1000.0;
    p.synchronization_ns = kLaunchNs;
    const double rows = static_cast<double>(w.rows), cols = static_cast<double>(w.cols);
    const double nnz = static_cast<double>(w.nnz), n = static_cast<double>(w.out_cols);
    if (core::same_stable_id(candidate, quantized_csr_candidate_id)) {
        if (w.out_cols == 0u) return false;
        const double code_bytes = w.bits != 0u ? nnz * w.bits / 8.0 : nnz * w.value_bytes;
        const double bytes = (rows + 1.0) * 8.0 + nnz * 4.0 + code_bytes + cols * (n * 2.0 + 8.0) + rows * n * 4.0;
        const double flops = 2.0 * nnz * n;
        p.kernel_ns = std::max(bytes / kHbmBytesPerNs, flops / kValuFlopsPerNs) / kQcsrEfficiency;
        // one-time column-order check and metadata interleave
        p.backend_prepare_ns = (nnz * 4.0 + rows * 8.0) / kHbmBytesPerNs + kLaunchNs;
        p.persistent_bytes = static_cast<std::uint64_t>(bytes - rows * n * 4.0 - cols * n * 2.0);
        p.transient_bytes = 0u;
    } else if (core::same_stable_id(candidate, quantized_csr_execution_order_candidate_id)) {
        if (w.out_cols == 0u || w.bits == 0u) return false;
        const double head = static_cast<double>(std::min<std::uint64_t>(
            w.head_genes != 0u ? w.head_genes : 2048u, w.cols / 1024u * 1024u));
        const double flops = 2.0 * nnz * n;
        const double code_bytes = nnz * w.bits / 8.0;
        const double structure_bytes = (rows + 1.0) * 8.0 + nnz * 4.0 + code_bytes + cols * 8.0;
        p.kernel_ns = flops / kValuFlopsPerNs / kQcsrExecEfficiency;
        // popularity order, relabel, dense head, tail stream (plan and fill)
        p.backend_prepare_ns = nnz * kQcsrExecPrepareNsPerEntry + 4.0 * kLaunchNs;
        // head: one byte per (row, head gene) in table form (codes and presence bits in words
        // form); tail stream: about 1.3 padded entries per tail entry, taken as half the entries
        const double head_bytes = w.bits <= 4u ? rows * head : rows * head * (w.bits + 1.0) / 8.0;
        const double stream_bytes = 0.5 * nnz * 1.3 * (w.bits == 8u ? 4.0 : 2.0) + rows * 28.0;
        p.persistent_bytes = static_cast<std::uint64_t>(structure_bytes + head_bytes + stream_bytes + cols * 12.0);
        // W in execution order, the head's partial sums, the head's weight panel
        p.transient_bytes = static_cast<std::uint64_t>(align256d(cols * n * 2.0) + align256d(rows * 256.0)
                                                       + align256d(head * n * 2.0));
    } else if (core::same_stable_id(candidate, blocked_ell_candidate_id)) {
        if (w.out_cols == 0u || w.block_size == 0u || w.ell_columns == 0u) return false;
        const double slots = rows * static_cast<double>(w.ell_columns);
        const double index_bytes = rows / w.block_size * (static_cast<double>(w.ell_columns) / w.block_size) * 4.0;
        const double bytes = slots * w.value_bytes + index_bytes + cols * n * 2.0 + rows * n * 4.0;
        const double flops = 2.0 * slots * n;
        p.kernel_ns = std::max(bytes / kHbmBytesPerNs, flops / kMfmaFlopsPerNs) / kBellEfficiency;
        // the weight panel is packed once per weight generation
        p.backend_prepare_ns = cols * n * 4.0 / kHbmBytesPerNs + kLaunchNs;
        p.persistent_bytes = static_cast<std::uint64_t>(slots * w.value_bytes + index_bytes + cols * n * 2.0);
        p.transient_bytes = static_cast<std::uint64_t>(cols * n * 2.0);  // repack workspace without a panel
    } else if (core::same_stable_id(candidate, cpbp_candidate_id)) {
        const double bytes = nnz * w.value_bytes + static_cast<double>(w.tile_blocks) * 16.0 + cols * 4.0 + rows * 8.0;
        p.kernel_ns = bytes / kHbmBytesPerNs / kCpbpEfficiency;
        p.backend_prepare_ns = 0.0;
        p.persistent_bytes = static_cast<std::uint64_t>(bytes - rows * 4.0);
    } else {
        return false;
    }
    p.kernel_ns += kLaunchNs;
    *out = p;
    return true;
}

bool planner_candidate_for(const core::operation_candidate &operation, const core::projection_key &projection,
                           const workload_shape &shape, cellerator::planner::planner_candidate *out) noexcept {
    if (out == nullptr) return false;
    cellerator::planner::planner_candidate c{};
    c.identity = operation.identity;
    c.name = operation.name;
    c.operation = &operation;
    c.projection = projection;
    if (!analytical_costs(operation.identity, shape, &c.analytical)) return false;
    c.flags = cellerator::planner::planner_candidate_correct;
    if ((operation.capability_flags & core::candidate_deterministic) != 0u)
        c.flags |= cellerator::planner::planner_candidate_deterministic;
    if ((operation.capability_flags & core::candidate_graph_capture) != 0u)
        c.flags |= cellerator::planner::planner_candidate_graph_capture;
    *out = c;
    return true;
}

const char *last_engine_error() noexcept { return engine_error; }

} // namespace cellerator_amd::cpmath
