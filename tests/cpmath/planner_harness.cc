// Test harness: runs the reference's own end-to-end planner
// (src/planner/end_to_end_planner.cc, compiled from its source into oracle/_ref/ by
// oracle/Makefile) over the engine's CP-Math candidates, the way a Cellerator host plans a
// projection: planner candidates from the engine's operation candidates and analytical
// phases (cpmath::planner_candidate_for), the host's policy, an optional measurement hook
// (forwarded to a C callback the Python tests provide, which runs the real kernels) and an
// optional single-entry plan cache kept in this library.
#include <cellerator_amd/cpmath/cpmath_backend.hh>

#include <cstdint>
#include <cstring>

namespace core = cellerator::compute::math::core;
namespace ex = cellerator::execution;
namespace pl = cellerator::planner;
namespace cp = cellerator_amd::cpmath;

extern "C" {

typedef struct ph_measurement {
    int32_t ok, correct, contaminated;
    uint32_t samples;
    double kernel_ns;
    double spread_percent;
} ph_measurement;

typedef int (*ph_measure_fn)(uint64_t id_low, uint64_t id_high, ph_measurement *out);

typedef struct ph_case {
    uint64_t rows, cols, nnz;
    uint32_t out_cols, bits, value_bytes, block_size;
    uint64_t ell_columns, tile_blocks;
    uint32_t problem_kind;   // 1 sparse_dense_multiply, 2 weighted_relation_reduce
    uint32_t candidate_mask; // bit 0 quantized CSR, bit 1 Blocked-ELL, bit 2 CP-BP, bit 3 execution-order CSR
    uint32_t deterministic, graph_capture_required;
    uint64_t max_persistent, max_transient;
    uint32_t shortlist, max_measurements;
    uint64_t min_tuning_work_items, logical_work_items;
    uint64_t structure_reuse, projection_reuse;
    double practical_tolerance, max_spread, min_cache_confidence;
    uint32_t allow_fallback, tune_one_shot;
    uint32_t nondeterministic_mask;  // candidates (same bits) to present without the deterministic flag
    uint32_t use_cache;              // 0 none, 1 lookup + store in the harness cache, 2 also clear it first
    ph_measure_fn measure;
    uint64_t evidence_revision;
} ph_case;

typedef struct ph_diag {
    uint64_t id_low, id_high;
    uint32_t rejection, shortlisted, measured, conventional;
    double analytical_ns, empirical_ns;
} ph_diag;

typedef struct ph_result {
    int32_t status;
    uint32_t source, cache, tuning_skipped, conventional_winner, legal, shortlist, measured;
    uint64_t winner_low, winner_high;
    double confidence;
    uint32_t count, stored;
    ph_diag diags[4];
    char reason[160];
    char message[160];
} ph_result;

int ph_case_size(void) { return (int)sizeof(ph_case); }
int ph_result_size(void) { return (int)sizeof(ph_result); }

}  // extern "C"

namespace {

struct hook_context {
    ph_measure_fn measure;
    const pl::planner_candidate *candidates;
    uint32_t count;
};

bool measure_trampoline(void *context, const pl::planner_candidate &candidate,
                        pl::measured_candidate *out) noexcept {
    auto *h = static_cast<hook_context *>(context);
    ph_measurement m{};
    if (h->measure(candidate.identity.low, candidate.identity.high, &m) != 0 || m.ok == 0) return false;
    *out = {};
    out->correct = m.correct != 0;
    out->contaminated = m.contaminated != 0;
    out->sample_count = m.samples;
    out->spread_percent = m.spread_percent;
    out->phases = candidate.analytical;  // every phase as modelled but the kernel, which is measured
    out->phases.kernel_ns = m.kernel_ns;
    return true;
}

pl::plan_cache_entry g_cache{};
bool g_cache_full = false;

bool cache_lookup(void *, const pl::planning_keys &, pl::plan_cache_entry *entry) noexcept {
    if (!g_cache_full) return false;
    *entry = g_cache;
    return true;
}

bool cache_store(void *, const pl::plan_cache_entry &entry) noexcept {
    g_cache = entry;
    g_cache_full = true;
    return true;
}

pl::planning_keys make_keys(const ph_case *c) {
    pl::planning_keys k{};
    k.problem.identity = {0x71u, 0x72u};
    core::structure_set_key live{};
    live.count = 1u;
    live.structures[0] = {{0x51u, 0x52u}, {5u, 1u}, {7u}};
    (void)pl::make_persistent_structure_set_key(live, &k.structures);
    k.geometry = {{2u, 3u}, {3u, 4u}, {4u, 5u}, {6u, 7u}, {8u, 9u}, {10u, 11u}};
    k.device = {0x1002u, 9u, 5u, 950u};  // AMD, gfx950
    k.build = {70200u, 1u, 1u, 1u};
    k.policy = {c->structure_reuse, c->projection_reuse, 1u, 1u, 1u, 1u};
    return k;
}

}  // namespace

extern "C" int ph_plan(const ph_case *c, ph_result *r) {
    std::memset(r, 0, sizeof(*r));
    static const core::operation_candidate ops[4] = {cp::quantized_csr_candidate(), cp::blocked_ell_candidate(),
                                                     cp::cpbp_candidate(),
                                                     cp::quantized_csr_execution_order_candidate()};
    const core::projection_kind kinds[4] = {core::projection_kind::csr, core::projection_kind::blocked_ell,
                                            core::projection_kind::native_row_masked, core::projection_kind::csr};
    cp::workload_shape shape{};
    shape.rows = c->rows;
    shape.cols = c->cols;
    shape.nnz = c->nnz;
    shape.out_cols = c->out_cols;
    shape.bits = c->bits;
    shape.value_bytes = c->value_bytes;
    shape.block_size = c->block_size;
    shape.ell_columns = c->ell_columns;
    shape.tile_blocks = c->tile_blocks;
    pl::planner_candidate candidates[4]{};
    uint32_t count = 0u;
    for (uint32_t i = 0; i < 4u; ++i) {
        if ((c->candidate_mask & (1u << i)) == 0u) continue;
        const core::projection_key key{{0x100u + i, 0x200u + i}, {0x300u + i, 1u}, kinds[i], cp::physical_view_schema,
                                       i == 0u || i == 3u ? c->bits : 0u};
        cp::workload_shape s = shape;
        if (i != 0u) s.out_cols = i == 2u ? 0u : shape.out_cols;
        if (!cp::planner_candidate_for(ops[i], key, s, &candidates[count])) {
            // a shape the cost model cannot price: presented with invalid costs, so the
            // planner rejects it as malformed
            candidates[count].identity = ops[i].identity;
            candidates[count].name = ops[i].name;
            candidates[count].operation = &ops[i];
            candidates[count].projection = key;
            candidates[count].analytical.kernel_ns = -1.0;
            candidates[count].flags = pl::planner_candidate_correct;
        }
        if ((c->nondeterministic_mask & (1u << i)) != 0u)
            candidates[count].flags &= ~static_cast<uint32_t>(pl::planner_candidate_deterministic);
        ++count;
    }
    pl::planner_request q{};
    q.problem.kind = c->problem_kind == 2u ? core::operation_kind::weighted_relation_reduce
                                           : core::operation_kind::sparse_dense_multiply;
    q.problem.operation = {0x71u, 0x72u};
    q.problem.input_count = 2u;
    q.problem.output_count = 1u;
    q.problem.logical_work_items = c->logical_work_items;
    q.keys = make_keys(c);
    q.candidates = candidates;
    q.candidate_count = count;
    q.policy.shortlist_size = c->shortlist;
    q.policy.maximum_measurements = c->max_measurements;
    q.policy.minimum_tuning_work_items = c->min_tuning_work_items;
    q.policy.maximum_persistent_bytes = c->max_persistent;
    q.policy.maximum_transient_bytes = c->max_transient;
    q.policy.practical_tolerance_percent = c->practical_tolerance;
    q.policy.maximum_spread_percent = c->max_spread;
    q.policy.minimum_cache_confidence = c->min_cache_confidence;
    q.policy.deterministic = c->deterministic != 0u;
    q.policy.graph_capture_required = c->graph_capture_required != 0u;
    q.policy.tune_one_shot = c->tune_one_shot != 0u;
    q.policy.allow_analytical_fallback_after_measurement_failure = c->allow_fallback != 0u;
    hook_context hook{c->measure, candidates, count};
    if (c->measure != nullptr) q.measurement = {&hook, measure_trampoline};
    if (c->use_cache == 2u) g_cache_full = false;
    if (c->use_cache != 0u) q.cache = {nullptr, cache_lookup, cache_store};
    q.current_evidence_revision = c->evidence_revision;

    static pl::planner_result res;  // large: diagnostics for 32 candidates
    const bool full_before = g_cache_full;
    const pl::planner_status st = pl::plan_end_to_end(q, &res);
    r->status = static_cast<int32_t>(st.code);
    r->source = static_cast<uint32_t>(res.source);
    r->cache = static_cast<uint32_t>(res.cache);
    r->tuning_skipped = res.tuning_skipped;
    r->conventional_winner = res.conventional_winner;
    r->legal = res.legal_count;
    r->shortlist = res.shortlist_count;
    r->measured = res.measurement_count;
    r->winner_low = res.winner.low;
    r->winner_high = res.winner.high;
    r->confidence = res.confidence;
    r->count = count;
    r->stored = (!full_before && g_cache_full) || (res.source == pl::selection_source::empirical && g_cache_full);
    for (uint32_t i = 0; i < count; ++i) {
        const pl::candidate_diagnostic &d = res.diagnostics[i];
        r->diags[i] = {d.identity.low, d.identity.high, static_cast<uint32_t>(d.rejection), d.shortlisted,
                       d.measured, d.conventional, d.analytical.amortized_total_ns, d.empirical.amortized_total_ns};
    }
    std::strncpy(r->reason, res.reason != nullptr ? res.reason : "", sizeof(r->reason) - 1u);
    std::strncpy(r->message, st.message != nullptr ? st.message : "", sizeof(r->message) - 1u);
    return 0;
}
