// bell_plan.cpp -- host planner that groups Blocked-ELL row blocks sharing block columns.
//
// A group is a run of row blocks whose lists of valid block columns (slot order, empty
// slots skipped) are prefixes of one another: every member's k-th valid block column equals
// the longest member's k-th. The grouped MFMA kernel then loads each weight-panel slice once
// per group instead of once per row block. Row blocks that share no prefix with a neighbour
// are left as singletons for the per-row-block kernel.
//
// Construction: sort row blocks by their valid-column list (lexicographic, shorter prefix
// first, ties by row block), then walk the sorted order and extend the current group while
// the next list extends the group's longest one. Deterministic for any thread count (single
// threaded; O(R log R * W) for R row blocks of W slots).
//
// Schedule (cx_bell_schedule_groups): the launch runs one unit (a group, or a single row
// block as a one-member group) per workgroup, and the dispatcher places workgroup i on XCD
// i % 8; the kernel maps workgroup i < 8 * per (per = units / 8) to unit
// (i % 8) * per + i / 8, so XCD x runs the contiguous range [x * per, (x + 1) * per). With the
// planner's order cut into equal-count ranges, the XCDs' shares of value blocks differed by
// up to 28% at C4 (modules of 24..64 block columns), and every XCD waits on the heaviest.
// The schedule deals the units out so that every range carries about the same number of
// value blocks, while units of one module (same first block column) stay in one range where
// they fit, so their shared panel slices stay in that XCD's L2.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <numeric>
#include <vector>

#include "cellerator_amd.h"

namespace {

constexpr std::uint32_t kInvalid = 0xffffffffu;

thread_local char g_plan_error[256] = "";

int plan_fail(int status, const char *message) {
    std::strncpy(g_plan_error, message, sizeof(g_plan_error) - 1u);
    g_plan_error[sizeof(g_plan_error) - 1u] = '\0';
    return status;
}

} // namespace

extern "C" int cx_bell_plan_groups(const uint32_t *block_col_idx, uint32_t row_blocks,
                                   uint32_t slots, uint32_t max_group, uint32_t *order,
                                   uint32_t *group_offsets, uint32_t *group_count,
                                   uint32_t *single_count) {
    g_plan_error[0] = '\0';
    if (order == nullptr || group_offsets == nullptr || group_count == nullptr
        || single_count == nullptr || (row_blocks != 0u && block_col_idx == nullptr))
        return plan_fail(CX_STATUS_INVALID_ARGUMENT, "cx_bell_plan_groups: null argument");
    if (max_group == 0u || max_group > 4u)
        return plan_fail(CX_STATUS_INVALID_SHAPE, "cx_bell_plan_groups: max_group must be 1..4");
    // valid-column lists, in slot order
    std::vector<std::uint32_t> list_begin(row_blocks + 1u, 0u);
    std::vector<std::uint32_t> cols;
    cols.reserve(static_cast<std::size_t>(row_blocks) * slots);
    for (std::uint32_t rb = 0; rb < row_blocks; ++rb) {
        const std::uint32_t *row = block_col_idx + static_cast<std::size_t>(rb) * slots;
        for (std::uint32_t s = 0; s < slots; ++s)
            if (row[s] != kInvalid) cols.push_back(row[s]);
        list_begin[rb + 1u] = static_cast<std::uint32_t>(cols.size());
    }
    auto length = [&](std::uint32_t rb) { return list_begin[rb + 1u] - list_begin[rb]; };
    auto at = [&](std::uint32_t rb, std::uint32_t k) { return cols[list_begin[rb] + k]; };
    std::vector<std::uint32_t> sorted(row_blocks);
    std::iota(sorted.begin(), sorted.end(), 0u);
    std::stable_sort(sorted.begin(), sorted.end(), [&](std::uint32_t x, std::uint32_t y) {
        const std::uint32_t lx = length(x), ly = length(y), l = std::min(lx, ly);
        for (std::uint32_t k = 0; k < l; ++k)
            if (at(x, k) != at(y, k)) return at(x, k) < at(y, k);
        return lx < ly;
    });
    // `longest` extends every other member: true when `shorter` is a prefix of `longer`
    auto is_prefix = [&](std::uint32_t shorter, std::uint32_t longer) {
        const std::uint32_t ls = length(shorter);
        if (ls > length(longer)) return false;
        for (std::uint32_t k = 0; k < ls; ++k)
            if (at(shorter, k) != at(longer, k)) return false;
        return true;
    };
    std::vector<std::vector<std::uint32_t>> groups;
    std::vector<std::uint32_t> singles;
    std::size_t i = 0;
    while (i < sorted.size()) {
        std::vector<std::uint32_t> g{sorted[i]};
        std::size_t k = i + 1;
        while (k < sorted.size() && g.size() < max_group && length(sorted[k]) != 0u
               && length(g.back()) != 0u && is_prefix(g.back(), sorted[k])) {
            g.push_back(sorted[k]);
            ++k;
        }
        if (g.size() >= 2u) groups.push_back(std::move(g));
        else singles.push_back(g[0]);
        i = k;
    }
    std::uint32_t pos = 0;
    for (std::size_t gi = 0; gi < groups.size(); ++gi) {
        group_offsets[gi] = pos;
        // the longest member last: it defines the group's column sequence
        for (std::uint32_t rb : groups[gi]) order[pos++] = rb;
    }
    group_offsets[groups.size()] = pos;
    for (std::uint32_t rb : singles) order[pos++] = rb;
    *group_count = static_cast<std::uint32_t>(groups.size());
    *single_count = static_cast<std::uint32_t>(singles.size());
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_bell_schedule_groups(const uint32_t *block_col_idx, uint32_t row_blocks, uint32_t slots,
                                       const uint32_t *order, const uint32_t *group_offsets,
                                       uint32_t group_count, uint32_t single_count,
                                       uint32_t *sched_order, uint32_t *sched_offsets,
                                       uint32_t *unit_count) {
    g_plan_error[0] = '\0';
    if (sched_offsets == nullptr || unit_count == nullptr
        || (row_blocks != 0u && (sched_order == nullptr || block_col_idx == nullptr || order == nullptr))
        || (group_count != 0u && group_offsets == nullptr))
        return plan_fail(CX_STATUS_INVALID_ARGUMENT, "cx_bell_schedule_groups: null argument");
    const std::uint32_t grouped = group_count != 0u ? group_offsets[group_count] : 0u;
    if (static_cast<std::uint64_t>(grouped) + single_count != row_blocks
        || (group_count != 0u && group_offsets[0] != 0u))
        return plan_fail(CX_STATUS_INVALID_SHAPE, "cx_bell_schedule_groups: the plan does not cover the row blocks");
    // units: (first member position in `order`, member count)
    const std::uint32_t units = group_count + single_count;
    std::vector<std::uint32_t> u_begin(units), u_size(units);
    std::vector<char> seen(row_blocks, 0);
    for (std::uint32_t g = 0; g < group_count; ++g) {
        if (group_offsets[g + 1u] <= group_offsets[g] || group_offsets[g + 1u] - group_offsets[g] > 4u)
            return plan_fail(CX_STATUS_INVALID_SHAPE, "cx_bell_schedule_groups: a group holds 1..4 row blocks");
        u_begin[g] = group_offsets[g];
        u_size[g] = group_offsets[g + 1u] - group_offsets[g];
    }
    for (std::uint32_t k = 0; k < single_count; ++k) {
        u_begin[group_count + k] = grouped + k;
        u_size[group_count + k] = 1u;
    }
    for (std::uint32_t i = 0; i < row_blocks; ++i) {
        if (order[i] >= row_blocks || seen[order[i]])
            return plan_fail(CX_STATUS_INVALID_SHAPE, "cx_bell_schedule_groups: order is not a permutation");
        seen[order[i]] = 1;
    }
    auto valid_count = [&](std::uint32_t rb) {
        const std::uint32_t *row = block_col_idx + static_cast<std::size_t>(rb) * slots;
        std::uint32_t n = 0;
        for (std::uint32_t s = 0; s < slots; ++s) n += row[s] != kInvalid ? 1u : 0u;
        return n;
    };
    auto first_col = [&](std::uint32_t rb) {
        const std::uint32_t *row = block_col_idx + static_cast<std::size_t>(rb) * slots;
        for (std::uint32_t s = 0; s < slots; ++s)
            if (row[s] != kInvalid) return row[s];
        return kInvalid;
    };
    // cost of a unit: its value blocks (the bytes its members stream); module key: the
    // leader's first block column
    std::vector<std::uint64_t> cost(units);
    std::vector<std::uint32_t> key(units);
    for (std::uint32_t u = 0; u < units; ++u) {
        std::uint64_t c = 0;
        for (std::uint32_t k = 0; k < u_size[u]; ++k) c += valid_count(order[u_begin[u] + k]);
        cost[u] = c;
        key[u] = first_col(order[u_begin[u] + u_size[u] - 1u]);
    }
    std::vector<std::uint32_t> logical(units);  // logical position -> unit
    constexpr std::uint32_t kXcds = 8;
    const std::uint32_t per = units / kXcds, full = per * kXcds;
    // units by module, then plan position (groups before singles within a module)
    std::vector<std::uint32_t> byk(units);
    std::iota(byk.begin(), byk.end(), 0u);
    std::stable_sort(byk.begin(), byk.end(), [&](std::uint32_t x, std::uint32_t y) { return key[x] < key[y]; });
    // the ragged tail (workgroups >= full keep their index) takes the cheapest units
    std::vector<std::uint32_t> by_cost(units);
    std::iota(by_cost.begin(), by_cost.end(), 0u);
    std::stable_sort(by_cost.begin(), by_cost.end(), [&](std::uint32_t x, std::uint32_t y) { return cost[x] < cost[y]; });
    std::vector<char> in_tail(units, 0);
    for (std::uint32_t k = 0; k < units - full; ++k) in_tail[by_cost[k]] = 1;
    {
        std::uint32_t t = full;
        for (std::uint32_t u : byk)
            if (in_tail[u]) logical[t++] = u;
    }
    if (per != 0u) {
        // modules (runs of one key), heaviest first, each to the lightest range with room
        std::vector<std::vector<std::uint32_t>> chunks;
        for (std::uint32_t u : byk) {
            if (in_tail[u]) continue;
            if (chunks.empty() || key[chunks.back().back()] != key[u]) chunks.emplace_back();
            chunks.back().push_back(u);
        }
        std::vector<std::uint64_t> chunk_cost(chunks.size(), 0);
        for (std::size_t c = 0; c < chunks.size(); ++c)
            for (std::uint32_t u : chunks[c]) chunk_cost[c] += cost[u];
        std::vector<std::uint32_t> corder(chunks.size());
        std::iota(corder.begin(), corder.end(), 0u);
        std::stable_sort(corder.begin(), corder.end(),
                         [&](std::uint32_t x, std::uint32_t y) { return chunk_cost[x] > chunk_cost[y]; });
        std::vector<std::vector<std::uint32_t>> range(kXcds);
        std::vector<std::uint64_t> work(kXcds, 0);
        for (std::uint32_t c : corder) {
            std::size_t next = 0;
            while (next < chunks[c].size()) {
                std::uint32_t best = kXcds;
                for (std::uint32_t x = 0; x < kXcds; ++x)
                    if (range[x].size() < per && (best == kXcds || work[x] < work[best])) best = x;
                const std::size_t take = std::min<std::size_t>(per - range[best].size(), chunks[c].size() - next);
                for (std::size_t k = 0; k < take; ++k) {
                    range[best].push_back(chunks[c][next + k]);
                    work[best] += cost[chunks[c][next + k]];
                }
                next += take;
            }
        }
        // refine: swap one unit of the heaviest range with one of the lightest, the pair whose
        // cost difference comes closest to half the gap, until no swap narrows it
        for (std::uint32_t it = 0; it < 4u * units; ++it) {
            std::uint32_t xa = 0, xb = 0;
            for (std::uint32_t x = 1; x < kXcds; ++x) {
                if (work[x] > work[xa]) xa = x;
                if (work[x] < work[xb]) xb = x;
            }
            const std::uint64_t gap = work[xa] - work[xb];
            if (gap < 2u) break;
            std::vector<std::uint32_t> light(range[xb]);
            std::stable_sort(light.begin(), light.end(), [&](std::uint32_t x, std::uint32_t y) { return cost[x] < cost[y]; });
            std::size_t bi = 0, bj = 0;
            std::uint64_t bd = 0;
            for (std::size_t i = 0; i < range[xa].size(); ++i) {
                const std::uint64_t ca = cost[range[xa][i]];
                // light unit with cost closest to ca - gap / 2, below ca
                const std::uint64_t want = ca > gap / 2u ? ca - gap / 2u : 0u;
                const auto pos = std::lower_bound(light.begin(), light.end(), want,
                                                  [&](std::uint32_t u, std::uint64_t v) { return cost[u] < v; });
                for (int side = 0; side < 2; ++side) {
                    const auto q = side == 0 ? pos : pos - 1;
                    if (q < light.begin() || q >= light.end() || cost[*q] >= ca) continue;
                    const std::uint64_t d = ca - cost[*q];
                    if (d >= gap) continue;
                    const auto dist = [&](std::uint64_t v) { return v > gap / 2u ? v - gap / 2u : gap / 2u - v; };
                    if (bd == 0u || dist(d) < dist(bd)) {
                        bd = d;
                        bi = i;
                        bj = static_cast<std::size_t>(std::find(range[xb].begin(), range[xb].end(), *q) - range[xb].begin());
                    }
                }
            }
            if (bd == 0u) break;
            std::swap(range[xa][bi], range[xb][bj]);
            work[xa] -= bd;
            work[xb] += bd;
        }
        for (std::uint32_t x = 0; x < kXcds; ++x)
            for (std::uint32_t j = 0; j < per; ++j) logical[x * per + j] = range[x][j];
    }
    std::uint32_t pos = 0;
    for (std::uint32_t l = 0; l < units; ++l) {
        const std::uint32_t u = logical[l];
        sched_offsets[l] = pos;
        for (std::uint32_t k = 0; k < u_size[u]; ++k) sched_order[pos++] = order[u_begin[u] + k];
    }
    sched_offsets[units] = pos;
    *unit_count = units;
    return CX_STATUS_SUCCESS;
}

extern "C" const char *cx_bell_plan_last_error(void) { return g_plan_error; }
