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

extern "C" const char *cx_bell_plan_last_error(void) { return g_plan_error; }
