// spmm_request.cpp -- the backend-neutral SpMM request on the host: validation
// (src/compute/math/operation.cc:119-293), the 128-bit operation signature
// (src/compute/math/operation_signature.cc:1-70), the trivial-work classification, and a
// request-driven entry onto the quantized CSR kernels.
//
// The checks run in the reference's order and return its codes and messages, because a
// caller compares them; the signature's splitmix64 chain and seeds are the reference's,
// because signatures are plan-cache keys shared across implementations (a fixed request has
// a fixed signature, pinned by the reference's own test vector).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <limits>

#include "cellerator_amd.h"
#include "cx_common.hpp"

namespace {

using u32 = std::uint32_t;
using u64 = std::uint64_t;

bool known_type(u32 c) { return c >= CX_REAL_F16 && c <= CX_REAL_FP8_E5M2; }
bool known_transpose(u32 v) { return v == CX_TRANSPOSE_NONE || v == CX_TRANSPOSE; }
bool known_layout(u32 v) { return v == CX_LAYOUT_ROW_MAJOR || v == CX_LAYOUT_COLUMN_MAJOR; }
bool known_determinism(u32 v) { return v == CX_ALLOW_NONDETERMINISTIC || v == CX_DETERMINISTIC; }
bool known_workspace(u32 v) { return v >= CX_WORKSPACE_REUSABLE_POOL && v <= CX_WORKSPACE_NONE; }
bool known_reuse(u32 v) { return v >= CX_REUSE_SINGLE_RUN && v <= CX_REUSE_PERSISTENT; }
bool known_epilogue(u32 v) { return v <= CX_EPILOGUE_BIAS_GELU_TANH; }
bool bias_kind(u32 v) {
    return v == CX_EPILOGUE_BIAS || v == CX_EPILOGUE_BIAS_RELU || v == CX_EPILOGUE_BIAS_GELU_ERF
        || v == CX_EPILOGUE_BIAS_GELU_TANH;
}

// An f32 scalar keeps the high word zero; f64 is any bit pattern.
bool canonical_scalar(const cx_scalar_value &v) {
    if (v.reserved != 0u) return false;
    if (v.type_code == CX_REAL_F32) return (v.bits >> 32u) == 0u;
    return v.type_code == CX_REAL_F64;
}

bool scalar_zero(const cx_scalar_value &v) {
    if (v.type_code == CX_REAL_F32) {
        float f;
        const u32 lo = static_cast<u32>(v.bits);
        std::memcpy(&f, &lo, 4);
        return f == 0.0f;
    }
    if (v.type_code == CX_REAL_F64) {
        double d;
        std::memcpy(&d, &v.bits, 8);
        return d == 0.0;
    }
    return false;
}

bool same_order(const cx_feature_order_identity &a, const cx_feature_order_identity &b) {
    return a.schema_version == b.schema_version && a.kind == b.kind && a.feature_count == b.feature_count
        && a.feature_axis_identity_version == b.feature_axis_identity_version
        && a.feature_axis_identity == b.feature_axis_identity
        && a.packing_geometry_identity == b.packing_geometry_identity;
}

u32 result(const char **message, u32 code, const char *text) {
    if (message != nullptr) *message = text;
    return code;
}

u32 validate(const cx_spmm_request &r, const char **msg) {
    if (r.schema_version != CX_OPERATION_CONTRACT_SCHEMA_VERSION || r.operation != CX_OPERATION_SPMM)
        return result(msg, CX_REQUEST_UNSUPPORTED_VERSION, "unsupported SpMM operation contract");
    if (r.sparse_nnz != 0u && (r.m == 0u || r.k == 0u))
        return result(msg, CX_REQUEST_INVALID_SHAPE, "nonzero sparse_nnz requires nonzero M and K");
    constexpr u64 kMax = std::numeric_limits<u64>::max();
    const bool mk = r.m != 0u && r.k > kMax / r.m;
    const bool mn = r.m != 0u && r.n > kMax / r.m;
    const bool kn = r.k != 0u && r.n > kMax / r.k;
    if (mk || kn || mn || r.sparse_nnz > r.m * r.k)
        return result(msg, CX_REQUEST_INVALID_SHAPE, "SpMM shape or sparse_nnz exceeds the addressable logical matrix");
    if (!known_transpose(r.transpose_sparse) || !known_transpose(r.transpose_dense))
        return result(msg, CX_REQUEST_INVALID_LAYOUT, "SpMM request contains an unknown transpose mode");
    if (!known_layout(r.dense_rhs_layout) || !known_layout(r.output_layout))
        return result(msg, CX_REQUEST_INVALID_LAYOUT, "unknown SpMM dense layout");
    // the dense operand as stored: K x N, or N x K when transposed
    const u64 rhs_rows = r.transpose_dense == CX_TRANSPOSE_NONE ? r.k : r.n;
    const u64 rhs_cols = r.transpose_dense == CX_TRANSPOSE_NONE ? r.n : r.k;
    const u64 rhs_min = r.dense_rhs_layout == CX_LAYOUT_ROW_MAJOR ? rhs_cols : rhs_rows;
    const u64 out_min = r.output_layout == CX_LAYOUT_ROW_MAJOR ? r.n : r.m;
    if ((rhs_rows != 0u && rhs_cols != 0u && r.dense_rhs_leading_dimension < rhs_min)
        || (r.m != 0u && r.n != 0u && r.output_leading_dimension < out_min))
        return result(msg, CX_REQUEST_INVALID_LAYOUT, "dense leading dimension is smaller than its physical matrix");
    if (!known_type(r.sparse_storage_type_code) || !known_type(r.dense_storage_type_code)
        || !known_type(r.output_storage_type_code) || !known_type(r.compute_type_code)
        || !known_type(r.accumulation_type_code))
        return result(msg, CX_REQUEST_INVALID_TYPE, "SpMM request contains an unknown numeric type code");
    if (r.alpha.type_code != r.compute_type_code || r.beta.type_code != r.compute_type_code
        || !canonical_scalar(r.alpha) || !canonical_scalar(r.beta))
        return result(msg, CX_REQUEST_INVALID_SCALAR,
                      "alpha and beta must use canonical request-compute f32 or f64 values");
    if (!known_determinism(r.determinism))
        return result(msg, CX_REQUEST_INVALID_DETERMINISM, "SpMM request contains an unknown determinism requirement");
    const cx_workspace_policy &w = r.workspace;
    if (!known_workspace(w.kind) || w.reserved != 0u || (w.kind == CX_WORKSPACE_CALLER_LIMIT) != (w.byte_limit != 0u))
        return result(msg, CX_REQUEST_INVALID_WORKSPACE_POLICY, "workspace kind and byte limit disagree");
    const cx_expected_reuse &u = r.reuse;
    if (!known_reuse(u.kind) || u.reserved != 0u
        || (u.kind == CX_REUSE_SINGLE_RUN && u.expected_run_count != 1u)
        || (u.kind == CX_REUSE_BOUNDED && u.expected_run_count == 0u)
        || (u.kind == CX_REUSE_PERSISTENT && u.expected_run_count != 0u))
        return result(msg, CX_REQUEST_INVALID_REUSE, "reuse kind and expected run count disagree");
    if (r.sparse_structure.schema_version != 1u || r.sparse_structure.identity_version == 0u
        || r.sparse_structure.value == 0u)
        return result(msg, CX_REQUEST_INVALID_IDENTITY, "SpMM request requires a stable sparse structure identity");
    auto order_ok = [&](const cx_feature_order_identity &o) {
        return o.schema_version == 1u && o.feature_count == r.k && o.feature_axis_identity != 0u
            && o.feature_axis_identity_version != 0u
            && ((o.kind == CX_FEATURE_ORDER_KIND_CANONICAL && o.packing_geometry_identity == 0u)
                || (o.kind == CX_FEATURE_ORDER_KIND_PACKED && o.packing_geometry_identity != 0u));
    };
    if (!order_ok(r.sparse_feature_order) || !order_ok(r.dense_feature_order))
        return result(msg, CX_REQUEST_INVALID_FEATURE_ORDER,
                      "SpMM feature-order identity is incomplete or disagrees with K");
    if (!same_order(r.sparse_feature_order, r.dense_feature_order))
        return result(msg, CX_REQUEST_FEATURE_ORDER_MISMATCH, "sparse and dense operands use different feature orders");
    if (!known_epilogue(r.epilogue.kind))
        return result(msg, CX_REQUEST_INVALID_EPILOGUE, "SpMM request contains an unknown epilogue");
    if (bias_kind(r.epilogue.kind)) {
        if (r.epilogue.bias_element_count != r.n || r.epilogue.bias_type_code != r.output_storage_type_code)
            return result(msg, CX_REQUEST_MISSING_BIAS, "bias epilogue requires N output-typed elements");
    } else if (r.epilogue.bias_element_count != 0u || r.epilogue.bias_type_code != 0u) {
        return result(msg, CX_REQUEST_UNEXPECTED_BIAS, "non-bias epilogue must not describe bias storage");
    }
    return result(msg, CX_REQUEST_OK, "ok");
}

u32 classify(const cx_spmm_request &r) {
    if (r.m == 0u || r.n == 0u) return CX_TRIVIAL_NO_OUTPUT;
    if (r.k == 0u || r.sparse_nnz == 0u || scalar_zero(r.alpha)) return CX_TRIVIAL_EPILOGUE_ONLY;
    return CX_TRIVIAL_NONE;
}

// splitmix64 finalizer and the two-lane mix of the signature.
constexpr u64 splitmix64(u64 x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30u)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27u)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31u);
}

struct Sig {
    u64 low = 0x43504d4154484f50ull;   // "CPMATHOP"
    u64 high = 0x53504d4d00000001ull;  // "SPMM", 1
    Sig &operator<<(u64 v) {
        low = splitmix64(low ^ v);
        high = splitmix64(high + v + 0x9e3779b97f4a7c15ull);
        return *this;
    }
    Sig &operator<<(const cx_feature_order_identity &o) {
        return *this << o.schema_version << o.kind << o.feature_count << o.feature_axis_identity_version
                     << o.feature_axis_identity << o.packing_geometry_identity;
    }
};

bool as_f32(const cx_scalar_value &v, float *out) {
    if (v.type_code == CX_REAL_F32) {
        const u32 lo = static_cast<u32>(v.bits);
        std::memcpy(out, &lo, 4);
        return true;
    }
    double d;
    std::memcpy(&d, &v.bits, 8);
    *out = static_cast<float>(d);
    return static_cast<double>(*out) == d || d != d;
}

} // namespace

static_assert(sizeof(cx_spmm_request) == 264, "cx_spmm_request must keep the reference's layout");
static_assert(sizeof(cx_feature_order_identity) == 32 && sizeof(cx_scalar_value) == 16, "identity layouts");

extern "C" void cx_spmm_request_init(cx_spmm_request *r) {
    if (r == nullptr) return;
    std::memset(r, 0, sizeof(*r));
    r->schema_version = CX_OPERATION_CONTRACT_SCHEMA_VERSION;
    r->operation = CX_OPERATION_SPMM;
    r->sparse_structure.schema_version = 1u;
    r->dense_rhs_layout = r->output_layout = CX_LAYOUT_ROW_MAJOR;
    r->workspace.kind = CX_WORKSPACE_REUSABLE_POOL;
    r->reuse.kind = CX_REUSE_SINGLE_RUN;
    r->reuse.expected_run_count = 1u;
    r->sparse_feature_order.schema_version = r->dense_feature_order.schema_version = 1u;
    r->sparse_feature_order.kind = r->dense_feature_order.kind = CX_FEATURE_ORDER_KIND_CANONICAL;
}

extern "C" cx_scalar_value cx_scalar_f32(float value) {
    cx_scalar_value s{};
    s.type_code = CX_REAL_F32;
    u32 b;
    std::memcpy(&b, &value, 4);
    s.bits = b;
    return s;
}

extern "C" cx_scalar_value cx_scalar_f64(double value) {
    cx_scalar_value s{};
    s.type_code = CX_REAL_F64;
    std::memcpy(&s.bits, &value, 8);
    return s;
}

extern "C" uint32_t cx_validate_spmm_request(const cx_spmm_request *request, const char **message) {
    if (request == nullptr) return result(message, CX_REQUEST_UNSUPPORTED_VERSION, "null request");
    return validate(*request, message);
}

extern "C" uint32_t cx_validate_math_request(const cx_spmm_request *request, const cx_spmm_bindings *bindings,
                                             const char **message) {
    if (request == nullptr || bindings == nullptr)
        return result(message, CX_REQUEST_MISSING_BINDING, "null request or bindings");
    const u32 code = validate(*request, message);
    if (code != CX_REQUEST_OK) return code;
    const u32 work = classify(*request);
    if (work == CX_TRIVIAL_NO_OUTPUT) return result(message, CX_REQUEST_OK, "ok");
    if (bindings->output == nullptr)
        return result(message, CX_REQUEST_MISSING_BINDING, "nonempty SpMM output requires an output binding");
    if (bias_kind(request->epilogue.kind)) {
        if (bindings->bias == nullptr)
            return result(message, CX_REQUEST_MISSING_BIAS, "bias epilogue requires a bias binding");
    } else if (bindings->bias != nullptr) {
        return result(message, CX_REQUEST_UNEXPECTED_BIAS, "non-bias epilogue received a bias binding");
    }
    if (work == CX_TRIVIAL_NONE && (bindings->sparse_matrix == nullptr || bindings->dense_rhs == nullptr))
        return result(message, CX_REQUEST_MISSING_BINDING, "nontrivial SpMM requires sparse and dense input bindings");
    return result(message, CX_REQUEST_OK, "ok");
}

extern "C" cx_operation_signature cx_make_operation_signature(const cx_spmm_request *request) {
    cx_operation_signature out{CX_OPERATION_CONTRACT_SCHEMA_VERSION, CX_OPERATION_SPMM, 0u, 0u};
    if (request == nullptr) return out;
    const cx_spmm_request &r = *request;
    Sig s;
    s << r.schema_version << r.operation << r.m << r.k << r.n << r.sparse_nnz << r.sparse_structure.schema_version
      << r.sparse_structure.identity_version << r.sparse_structure.value << r.transpose_sparse << r.transpose_dense
      << r.dense_rhs_layout << r.output_layout << r.dense_rhs_leading_dimension << r.output_leading_dimension
      << r.sparse_storage_type_code << r.dense_storage_type_code << r.output_storage_type_code << r.compute_type_code
      << r.accumulation_type_code << r.alpha.type_code << r.alpha.bits << r.beta.type_code << r.beta.bits
      << r.determinism << r.workspace.kind << r.workspace.byte_limit << r.reuse.kind << r.reuse.expected_run_count
      << r.epilogue.kind << r.epilogue.bias_type_code << r.epilogue.bias_element_count << r.sparse_feature_order
      << r.dense_feature_order;
    out.low = s.low;
    out.high = s.high;
    return out;
}

extern "C" uint32_t cx_classify_trivial_operation(const cx_spmm_request *request) {
    return request == nullptr ? CX_TRIVIAL_NO_OUTPUT : classify(*request);
}

namespace {

// Y = act(beta C + bias) with no product term (alpha 0, K 0 or no stored entries).
__global__ __launch_bounds__(256) void epilogue_only_kernel(cx::Epilogue e, std::uint64_t rows, std::int64_t cols,
                                                            float *out, std::int64_t ld) {
    const std::uint64_t total = rows * static_cast<std::uint64_t>(cols);
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
        const std::int64_t row = static_cast<std::int64_t>(i / static_cast<std::uint64_t>(cols));
        const std::int64_t col = static_cast<std::int64_t>(i % static_cast<std::uint64_t>(cols));
        out[row * ld + col] = cx::epilogue_value(e, 0.0f, row, col);
    }
}

} // namespace

extern "C" int cx_qcsr_spmm_fwd_request(const cx_spmm_request *request, const cx_spmm_bindings *bindings,
                                        void *stream) {
    using namespace cx;
    clear_error();
    const char *text = nullptr;
    if (cx_validate_math_request(request, bindings, &text) != CX_REQUEST_OK)
        return fail(CX_STATUS_INVALID_ARGUMENT, text);
    const cx_spmm_request &r = *request;
    const u32 work = classify(r);
    if (work == CX_TRIVIAL_NO_OUTPUT) return CX_STATUS_SUCCESS;
    if (r.transpose_sparse != CX_TRANSPOSE_NONE || r.transpose_dense != CX_TRANSPOSE_NONE
        || r.dense_rhs_layout != CX_LAYOUT_ROW_MAJOR || r.output_layout != CX_LAYOUT_ROW_MAJOR)
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_spmm_fwd_request: untransposed row-major operands only");
    if (r.output_storage_type_code != CX_REAL_F32 || r.compute_type_code != CX_REAL_F32
        || r.accumulation_type_code != CX_REAL_F32
        || (r.dense_storage_type_code != CX_REAL_F16 && r.dense_storage_type_code != CX_REAL_F32))
        return fail(CX_STATUS_UNSUPPORTED,
                    "cx_qcsr_spmm_fwd_request: F16 or F32 dense storage with F32 output, compute and accumulation");
    constexpr u64 kI64 = static_cast<u64>(std::numeric_limits<std::int64_t>::max());
    if (r.m > kI64 / (r.n == 0u ? 1u : r.n) || r.n > kI64 || r.output_leading_dimension > kI64
        || r.dense_rhs_leading_dimension > kI64)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_fwd_request: shape out of range");
    cx_spmm_epilogue ep{};
    ep.kind = r.epilogue.kind;
    if (!as_f32(r.alpha, &ep.alpha) || !as_f32(r.beta, &ep.beta))
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_spmm_fwd_request: alpha and beta must be exact in f32");
    auto *out = static_cast<float *>(bindings->output);
    const auto cols = static_cast<std::int64_t>(r.n);
    const auto out_ld = static_cast<std::int64_t>(r.output_leading_dimension);
    ep.bias = static_cast<const float *>(bindings->bias);
    ep.initial = ep.beta != 0.0f ? out : nullptr;
    ep.initial_ld = out_ld;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (work == CX_TRIVIAL_EPILOGUE_ONLY) {
        // the operands are neither needed nor read (the reference's epilogue-only semantics)
        ep.alpha = 0.0f;
        Epilogue dev;
        int rc = make_epilogue(&ep, r.m, cols, out, out_ld, &dev, "cx_qcsr_spmm_fwd_request");
        if (rc != CX_STATUS_SUCCESS) return rc;
        const u64 total = r.m * r.n;
        const unsigned blocks = static_cast<unsigned>(std::min<u64>((total + 255u) / 256u, 65536u));
        hipLaunchKernelGGL(epilogue_only_kernel, dim3(blocks), dim3(256), 0, s, dev, r.m, cols, out, out_ld);
        return check_launch("cx_qcsr_spmm_fwd_request");
    }
    const auto *a = static_cast<const cx_qcsr_matrix *>(bindings->sparse_matrix);
    if (a->rows != r.m || a->cols != r.k || a->nnz != r.sparse_nnz)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_fwd_request: the request does not describe the bound matrix");
    const u32 rhs_dtype = r.dense_storage_type_code == CX_REAL_F16 ? CELLERATOR_DTYPE_F16 : CELLERATOR_DTYPE_F32;
    return cx_qcsr_spmm_fwd_epilogue(a, bindings->dense_rhs, rhs_dtype,
                                     static_cast<int64_t>(r.dense_rhs_leading_dimension), cols, out, out_ld, &ep,
                                     stream);
}
