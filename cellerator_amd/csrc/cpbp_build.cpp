// cpbp_build.cpp -- host construction of the CP-BP warp-tile projection consumed by
// cx_cpbp_reduce: canonical CSR -> cell-block records -> local cell order -> warp tiles.
//
// Semantics follow the reference's host producers:
//   records : apply_frozen_plan_host + build_cell_block_records_host
//             (components/CellPack/src/apply_plan.cc:176-232,
//              components/CellPack/src/cell_block_records.cc:240-314): a row's entries
//             are ordered by (feature block, local feature) of the plan's execution
//             order; one record per (row, block) with a u32 gene mask and its values in
//             increasing local-feature order.
//   order   : build_local_cell_order_host (local_cell_ordering.cc:96-160,232-275):
//             per-row (primary, secondary) keys, stable sort inside each window of
//             window_size rows, ties broken by row index. inferred_minhash packs the top
//             16 bits of four splitmix64 minima over the row's block ids.
//   tiles   : build_warp_tiles_host (warp_tiles.cc:280-352): tile t = execution rows
//             [t*w, (t+1)*w); descriptors are the union of the lanes' blocks in
//             increasing block id; a descriptor's cell mask has one bit per lane that
//             holds the block; entries are compacted in lane order, values copied.
// Generalisation: tile widths 33..64 (the wave64 projection) store u64 cell masks; the
// reference limits widths to 32 with u32 masks (warp_tiles.cc:55).
//
// Windows (and the tiles inside them) are independent, so every stage runs on a pool of
// host threads over windows; offsets are joined with prefix sums, so the output is
// identical for any thread count.
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <new>
#include <thread>
#include <vector>

#include "cellerator_amd.h"

struct cx_cpbp_builder {
    cx_cpbp_tile_requirements req{};
    uint32_t value_size = 0u;
    uint32_t mask_bytes = 0u;
    std::vector<uint32_t> tile_block_offsets;
    std::vector<uint32_t> tile_block_ids;
    std::vector<uint64_t> cell_masks;  // widened; exported as u32 or u64
    std::vector<uint32_t> block_row_entry_offsets;
    std::vector<uint32_t> gene_masks;
    std::vector<uint32_t> value_offsets;
    std::vector<unsigned char> values;
    std::vector<uint32_t> row_permutation;
    std::vector<uint64_t> primary_keys;
    std::vector<uint32_t> secondary_keys;
};

namespace {

thread_local char g_build_error[256] = {0};

int fail(int status, const char *message) {
    std::snprintf(g_build_error, sizeof(g_build_error), "%s", message);
    return status;
}

uint64_t splitmix64(uint64_t value) {
    value += 0x9e3779b97f4a7c15ull;
    value = (value ^ (value >> 30u)) * 0xbf58476d1ce4e5b9ull;
    value = (value ^ (value >> 27u)) * 0x94d049bb133111ebull;
    return value ^ (value >> 31u);
}

constexpr uint32_t kInvalid = 0xffffffffu;
constexpr uint32_t kSignatureLanes = 4u;

// Runs fn(first, last) over [0, count) split into contiguous chunks on `threads` workers.
template<typename Fn>
void parallel_for(uint32_t count, uint32_t threads, Fn fn) {
    if (threads <= 1u || count < 2u) {
        fn(0u, count);
        return;
    }
    threads = std::min(threads, count);
    std::vector<std::thread> pool;
    pool.reserve(threads);
    const uint32_t per = count / threads, extra = count % threads;
    uint32_t begin = 0u;
    for (uint32_t t = 0u; t < threads; ++t) {
        const uint32_t end = begin + per + (t < extra ? 1u : 0u);
        pool.emplace_back([=] { fn(begin, end); });
        begin = end;
    }
    for (auto &th : pool) th.join();
}

struct PlanTables {
    std::vector<uint32_t> to_block;  // canonical feature -> block
    std::vector<uint32_t> to_local;  // canonical feature -> local bit
};

int check_plan(const cx_cpbp_plan *plan, PlanTables *t) {
    if (plan == nullptr || plan->feature_permutation == nullptr || plan->feature_block_offsets == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP plan has a null array");
    const uint32_t f = plan->feature_count, nb = plan->feature_block_count;
    if (nb == 0u && f != 0u) return fail(CX_STATUS_INVALID_SHAPE, "CP-BP plan has features but no blocks");
    if (plan->feature_block_offsets[0] != 0u || plan->feature_block_offsets[nb] != f)
        return fail(CX_STATUS_INVALID_SHAPE, "CP-BP plan block offsets must span [0, feature_count]");
    t->to_block.assign(f, kInvalid);
    t->to_local.assign(f, kInvalid);
    for (uint32_t b = 0u; b < nb; ++b) {
        const uint32_t lo = plan->feature_block_offsets[b], hi = plan->feature_block_offsets[b + 1u];
        if (hi <= lo || hi - lo > 32u)
            return fail(CX_STATUS_INVALID_SHAPE, "CP-BP plan feature blocks must hold 1..32 features");
        for (uint32_t e = lo; e < hi; ++e) {
            const uint32_t c = plan->feature_permutation[e];
            if (c >= f || t->to_block[c] != kInvalid)
                return fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP plan feature permutation is not a permutation");
            t->to_block[c] = b;
            t->to_local[c] = e - lo;
        }
    }
    return CX_STATUS_SUCCESS;
}

int check_csr(const cx_cpbp_csr *csr, uint32_t feature_count) {
    if (csr == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP source CSR is null");
    if (csr->value_size_bytes != 2u && csr->value_size_bytes != 4u)
        return fail(CX_STATUS_UNSUPPORTED, "CP-BP values must be 2-byte (f16) or 4-byte (f32)");
    if (csr->rows != 0u && csr->row_offsets == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP source row offsets are null");
    if (csr->rows == 0u) return CX_STATUS_SUCCESS;
    if (csr->row_offsets[0] != 0u) return fail(CX_STATUS_INVALID_SHAPE, "CP-BP source row offsets must start at zero");
    const uint32_t nnz = csr->row_offsets[csr->rows];
    if (nnz != 0u && (csr->canonical_features == nullptr || csr->values == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP source features or values are null");
    for (uint32_t r = 0u; r < csr->rows; ++r) {
        const uint32_t b = csr->row_offsets[r], e = csr->row_offsets[r + 1u];
        if (e < b || e > nnz) return fail(CX_STATUS_INVALID_SHAPE, "CP-BP source row offsets are not monotonic");
        for (uint32_t i = b; i < e; ++i) {
            const uint32_t feat = csr->canonical_features[i];
            if (feat >= feature_count)
                return fail(CX_STATUS_INVALID_SHAPE, "CP-BP source feature id is outside the feature axis");
            if (i > b && feat <= csr->canonical_features[i - 1u])
                return fail(CX_STATUS_INVALID_ARGUMENT,
                            "CP-BP source feature ids must be strictly increasing per row");
        }
    }
    return CX_STATUS_SUCCESS;
}

bool valid_kind(uint32_t kind) {
    return kind == CX_CPBP_ORDER_INFERRED_MINHASH || kind == CX_CPBP_ORDER_ORIGINAL
        || kind == CX_CPBP_ORDER_DETERMINISTIC_RANDOM || kind == CX_CPBP_ORDER_ROW_NNZ_DESCENDING;
}

// Per-row records in canonical row order.
struct Records {
    std::vector<uint32_t> row_offsets;   // rows + 1
    std::vector<uint32_t> block_ids;
    std::vector<uint32_t> gene_masks;
    std::vector<uint32_t> value_offsets; // records + 1
    std::vector<unsigned char> values;   // value_size per stored value, record order
};

void build_records(const cx_cpbp_csr *csr, const PlanTables &pt, uint32_t threads, Records *out) {
    const uint32_t rows = csr->rows, vs = csr->value_size_bytes;
    const uint32_t nnz = rows ? csr->row_offsets[rows] : 0u;
    // pass 1: records per row
    std::vector<uint32_t> count(rows + 1u, 0u);
    parallel_for(rows, threads, [&](uint32_t lo, uint32_t hi) {
        std::vector<uint64_t> keys;
        for (uint32_t r = lo; r < hi; ++r) {
            const uint32_t b = csr->row_offsets[r], e = csr->row_offsets[r + 1u];
            keys.clear();
            for (uint32_t i = b; i < e; ++i) keys.push_back(pt.to_block[csr->canonical_features[i]]);
            std::sort(keys.begin(), keys.end());
            count[r] = static_cast<uint32_t>(std::unique(keys.begin(), keys.end()) - keys.begin());
        }
    });
    out->row_offsets.assign(rows + 1u, 0u);
    for (uint32_t r = 0u; r < rows; ++r) out->row_offsets[r + 1u] = out->row_offsets[r] + count[r];
    const uint32_t nrec = out->row_offsets[rows];
    out->block_ids.assign(nrec, 0u);
    out->gene_masks.assign(nrec, 0u);
    out->value_offsets.assign(nrec + 1u, 0u);
    out->values.assign(static_cast<size_t>(nnz) * vs, 0u);
    const auto *src = static_cast<const unsigned char *>(csr->values);
    // pass 2: entries sorted by (block, local), stable in source order; values in that order
    parallel_for(rows, threads, [&](uint32_t lo, uint32_t hi) {
        std::vector<std::pair<uint64_t, uint32_t>> ent;
        for (uint32_t r = lo; r < hi; ++r) {
            const uint32_t b = csr->row_offsets[r], e = csr->row_offsets[r + 1u];
            ent.clear();
            for (uint32_t i = b; i < e; ++i) {
                const uint32_t c = csr->canonical_features[i];
                ent.emplace_back((static_cast<uint64_t>(pt.to_block[c]) << 32u) | pt.to_local[c], i);
            }
            std::stable_sort(ent.begin(), ent.end(),
                             [](const auto &x, const auto &y) { return x.first < y.first; });
            uint32_t rec = out->row_offsets[r] - 1u, cur = kInvalid;
            for (uint32_t k = 0u; k < ent.size(); ++k) {
                const uint32_t blk = static_cast<uint32_t>(ent[k].first >> 32u);
                const uint32_t loc = static_cast<uint32_t>(ent[k].first & 0xffffffffu);
                if (blk != cur) {
                    ++rec;
                    cur = blk;
                    out->block_ids[rec] = blk;
                    out->value_offsets[rec] = b + k;
                }
                out->gene_masks[rec] |= 1u << loc;
                std::memcpy(&out->values[static_cast<size_t>(b + k) * vs],
                            src + static_cast<size_t>(ent[k].second) * vs, vs);
            }
        }
    });
    out->value_offsets[nrec] = nnz;
}

void row_keys(const Records &rec, const cx_cpbp_order_config &cfg, uint32_t row, uint64_t *primary,
              uint32_t *secondary) {
    const uint32_t b = rec.row_offsets[row], e = rec.row_offsets[row + 1u];
    const uint32_t active = e - b;
    const uint32_t nnz = rec.value_offsets[e] - rec.value_offsets[b];
    *secondary = active;
    switch (cfg.kind) {
    case CX_CPBP_ORDER_INFERRED_MINHASH: {
        if (b == e) {
            *primary = std::numeric_limits<uint64_t>::max();
            break;
        }
        uint64_t packed = 0u;
        for (uint32_t lane = 0u; lane < kSignatureLanes; ++lane) {
            uint64_t minimum = std::numeric_limits<uint64_t>::max();
            const uint64_t lane_seed = splitmix64(cfg.seed ^ (static_cast<uint64_t>(lane) << 32u));
            for (uint32_t r = b; r < e; ++r)
                minimum = std::min(minimum, splitmix64(lane_seed ^ static_cast<uint64_t>(rec.block_ids[r])));
            packed = (packed << 16u) | ((minimum >> 48u) & 0xffffu);
        }
        *primary = packed;
        break;
    }
    case CX_CPBP_ORDER_ORIGINAL:
        *primary = row;
        *secondary = 0u;
        break;
    case CX_CPBP_ORDER_DETERMINISTIC_RANDOM:
        *primary = splitmix64(cfg.seed ^ (cfg.global_row_begin + row));
        *secondary = 0u;
        break;
    default:  // row_nnz_descending
        *primary = std::numeric_limits<uint64_t>::max() - nnz;
        break;
    }
}

} // namespace

extern "C" {

const char *cx_cpbp_build_last_error(void) { return g_build_error; }

int cx_cpbp_builder_create(const cx_cpbp_plan *plan, const cx_cpbp_csr *csr,
                           const cx_cpbp_order_config *config, uint32_t threads,
                           cx_cpbp_builder **out) {
    g_build_error[0] = '\0';
    if (out == nullptr || config == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP builder output or order config is null");
    *out = nullptr;
    PlanTables pt;
    int rc = check_plan(plan, &pt);
    if (rc != CX_STATUS_SUCCESS) return rc;
    rc = check_csr(csr, plan->feature_count);
    if (rc != CX_STATUS_SUCCESS) return rc;
    const cx_cpbp_order_config cfg = *config;
    if (!valid_kind(cfg.kind)) return fail(CX_STATUS_UNSUPPORTED, "local-cell order kind is unsupported");
    // local_cell_ordering.cc:23-35, plus the wave64 width limit of this engine
    if (cfg.window_size == 0u || cfg.group_width == 0u || cfg.group_width > cfg.window_size
        || cfg.window_size % cfg.group_width != 0u)
        return fail(CX_STATUS_INVALID_SHAPE, "local-cell windows must contain an integral nonzero number of groups");
    if (cfg.group_width > 64u) return fail(CX_STATUS_INVALID_SHAPE, "tile width must be at most 64 rows");
    if (threads == 0u) threads = 1u;

    cx_cpbp_builder *b = new (std::nothrow) cx_cpbp_builder();
    if (b == nullptr) return fail(CX_STATUS_INTERNAL_ERROR, "CP-BP builder allocation failed");
    try {
        const uint32_t rows = csr->rows, w = cfg.group_width, vs = csr->value_size_bytes;
        Records rec;
        build_records(csr, pt, threads, &rec);

        // ---- local order: keys, then a sort inside every window
        b->primary_keys.assign(rows, 0u);
        b->secondary_keys.assign(rows, 0u);
        b->row_permutation.resize(rows);
        const uint32_t windows = (rows + cfg.window_size - 1u) / cfg.window_size;
        parallel_for(windows, threads, [&](uint32_t lo, uint32_t hi) {
            for (uint32_t wi = lo; wi < hi; ++wi) {
                const uint32_t wb = wi * cfg.window_size;
                const uint32_t we = std::min(rows, wb + cfg.window_size);
                for (uint32_t r = wb; r < we; ++r) {
                    row_keys(rec, cfg, r, &b->primary_keys[r], &b->secondary_keys[r]);
                    b->row_permutation[r] = r;
                }
                std::sort(b->row_permutation.begin() + wb, b->row_permutation.begin() + we,
                          [&](uint32_t l, uint32_t r) {
                              if (b->primary_keys[l] != b->primary_keys[r])
                                  return b->primary_keys[l] < b->primary_keys[r];
                              if (b->secondary_keys[l] != b->secondary_keys[r])
                                  return b->secondary_keys[l] < b->secondary_keys[r];
                              return l < r;
                          });
            }
        });

        // ---- tiles: per-tile union of blocks; counts first, then fill at prefix offsets
        const uint32_t tiles = (rows + w - 1u) / w;
        std::vector<uint32_t> tblocks(tiles + 1u, 0u), tentries(tiles + 1u, 0u);
        auto walk = [&](uint32_t tile, auto &&emit) {
            const uint32_t tb = tile * w, lanes = std::min(w, rows - tb);
            uint32_t cur[64], end[64];
            for (uint32_t l = 0u; l < lanes; ++l) {
                const uint32_t canon = b->row_permutation[tb + l];
                cur[l] = rec.row_offsets[canon];
                end[l] = rec.row_offsets[canon + 1u];
            }
            while (true) {
                uint32_t block = kInvalid;
                for (uint32_t l = 0u; l < lanes; ++l)
                    if (cur[l] != end[l]) block = std::min(block, rec.block_ids[cur[l]]);
                if (block == kInvalid) break;
                uint64_t mask = 0u;
                uint32_t first = 0u, count = 0u;
                for (uint32_t l = 0u; l < lanes; ++l) {
                    if (cur[l] == end[l] || rec.block_ids[cur[l]] != block) continue;
                    if (count == 0u) first = cur[l];
                    mask |= uint64_t{1} << l;
                    emit(block, mask, l, cur[l], count);
                    ++cur[l];
                    ++count;
                }
                (void)first;
            }
        };
        parallel_for(tiles, threads, [&](uint32_t lo, uint32_t hi) {
            for (uint32_t t = lo; t < hi; ++t) {
                uint32_t nb = 0u, ne = 0u;
                uint32_t last_block = kInvalid;
                walk(t, [&](uint32_t block, uint64_t, uint32_t, uint32_t, uint32_t) {
                    if (block != last_block) { ++nb; last_block = block; }
                    ++ne;
                });
                tblocks[t + 1u] = nb;
                tentries[t + 1u] = ne;
            }
        });
        for (uint32_t t = 0u; t < tiles; ++t) {
            tblocks[t + 1u] += tblocks[t];
            tentries[t + 1u] += tentries[t];
        }
        const uint32_t nblocks = tblocks[tiles], nentries = tentries[tiles];
        const uint32_t nnz = rows ? csr->row_offsets[rows] : 0u;
        b->tile_block_offsets.assign(tblocks.begin(), tblocks.end());
        b->tile_block_ids.assign(nblocks, 0u);
        b->cell_masks.assign(nblocks, 0u);
        b->block_row_entry_offsets.assign(nblocks + 1u, 0u);
        b->gene_masks.assign(nentries, 0u);
        b->value_offsets.assign(nentries + 1u, 0u);
        b->values.assign(static_cast<size_t>(nnz) * vs, 0u);
        // value offsets of a tile start at the sum of its entries' value counts: a tile's
        // values are its rows' values, so the prefix over tiles is a prefix over row nnz
        std::vector<uint32_t> tvalues(tiles + 1u, 0u);
        for (uint32_t t = 0u; t < tiles; ++t) {
            uint32_t v = 0u;
            const uint32_t tb = t * w, lanes = std::min(w, rows - tb);
            for (uint32_t l = 0u; l < lanes; ++l) {
                const uint32_t canon = b->row_permutation[tb + l];
                v += rec.value_offsets[rec.row_offsets[canon + 1u]] - rec.value_offsets[rec.row_offsets[canon]];
            }
            tvalues[t + 1u] = tvalues[t] + v;
        }
        parallel_for(tiles, threads, [&](uint32_t lo, uint32_t hi) {
            for (uint32_t t = lo; t < hi; ++t) {
                uint32_t d = tblocks[t] - 1u, e = tentries[t], v = tvalues[t];
                uint32_t last_block = kInvalid;
                walk(t, [&](uint32_t block, uint64_t mask, uint32_t, uint32_t record, uint32_t) {
                    if (block != last_block) {
                        ++d;
                        last_block = block;
                        b->tile_block_ids[d] = block;
                        b->block_row_entry_offsets[d] = e;
                    }
                    b->cell_masks[d] = mask;
                    b->gene_masks[e] = rec.gene_masks[record];
                    b->value_offsets[e] = v;
                    const uint32_t vb = rec.value_offsets[record], ve = rec.value_offsets[record + 1u];
                    if (ve > vb)
                        std::memcpy(&b->values[static_cast<size_t>(v) * vs],
                                    &rec.values[static_cast<size_t>(vb) * vs],
                                    static_cast<size_t>(ve - vb) * vs);
                    v += ve - vb;
                    ++e;
                });
            }
        });
        b->block_row_entry_offsets[nblocks] = nentries;
        b->value_offsets[nentries] = nnz;
        b->value_size = vs;
        b->mask_bytes = w > 32u ? 8u : 4u;
        b->req.row_count = rows;
        b->req.feature_count = plan->feature_count;
        b->req.feature_block_count = plan->feature_block_count;
        b->req.tile_row_width = w;
        b->req.tile_count = tiles;
        b->req.tile_block_count = nblocks;
        b->req.row_block_entry_count = nentries;
        b->req.nnz_count = nnz;
        b->req.value_size_bytes = vs;
        b->req.cell_mask_bytes = b->mask_bytes;
    } catch (const std::bad_alloc &) {
        delete b;
        return fail(CX_STATUS_INTERNAL_ERROR, "CP-BP builder ran out of host memory");
    }
    *out = b;
    return CX_STATUS_SUCCESS;
}

int cx_cpbp_builder_requirements(const cx_cpbp_builder *b, cx_cpbp_tile_requirements *out) {
    if (b == nullptr || out == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "null builder or output");
    *out = b->req;
    return CX_STATUS_SUCCESS;
}

int cx_cpbp_builder_export(const cx_cpbp_builder *b, const cx_cpbp_tile_buffers *buf) {
    if (b == nullptr || buf == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "null builder or buffers");
    const cx_cpbp_tile_requirements &r = b->req;
    if (buf->tile_block_offsets == nullptr || buf->block_row_entry_offsets == nullptr
        || buf->row_block_value_offsets == nullptr
        || (r.row_count != 0u && buf->row_permutation == nullptr)
        || (r.tile_block_count != 0u && (buf->tile_block_ids == nullptr || buf->tile_block_cell_masks == nullptr))
        || (r.row_block_entry_count != 0u && buf->row_block_gene_masks == nullptr)
        || (r.nnz_count != 0u && buf->values == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "CP-BP export buffer is null");
    std::memcpy(buf->tile_block_offsets, b->tile_block_offsets.data(), (r.tile_count + 1u) * 4u);
    if (r.tile_block_count) std::memcpy(buf->tile_block_ids, b->tile_block_ids.data(), r.tile_block_count * 4u);
    if (b->mask_bytes == 8u) {
        if (r.tile_block_count)
            std::memcpy(buf->tile_block_cell_masks, b->cell_masks.data(), r.tile_block_count * 8u);
    } else {
        auto *m32 = static_cast<uint32_t *>(buf->tile_block_cell_masks);
        for (uint32_t d = 0u; d < r.tile_block_count; ++d) m32[d] = static_cast<uint32_t>(b->cell_masks[d]);
    }
    std::memcpy(buf->block_row_entry_offsets, b->block_row_entry_offsets.data(), (r.tile_block_count + 1u) * 4u);
    if (r.row_block_entry_count)
        std::memcpy(buf->row_block_gene_masks, b->gene_masks.data(), r.row_block_entry_count * 4u);
    std::memcpy(buf->row_block_value_offsets, b->value_offsets.data(), (r.row_block_entry_count + 1u) * 4u);
    if (r.nnz_count) std::memcpy(buf->values, b->values.data(), static_cast<size_t>(r.nnz_count) * b->value_size);
    if (r.row_count) std::memcpy(buf->row_permutation, b->row_permutation.data(), r.row_count * 4u);
    if (buf->primary_keys != nullptr && r.row_count)
        std::memcpy(buf->primary_keys, b->primary_keys.data(), r.row_count * 8u);
    return CX_STATUS_SUCCESS;
}

void cx_cpbp_builder_destroy(cx_cpbp_builder *b) { delete b; }

} // extern "C"
