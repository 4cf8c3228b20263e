// qcsr_stream.hip -- the prepared tail stream of an execution-order quantized CSR: the
// entries of every row from its first tail entry (head_end of the hybrid layout) on,
// rearranged once per structure into the order the row-group walk consumes them
// (qcsr_spmm_stream in qcsr_parts.hip), so the walk loads them instead of finding them.
//
// Geometry (qcsr_common.hpp): the rows are sorted by tail length over the whole matrix
// (descending, ties by row); sets of 8 consecutive rows of that order are dealt round-robin
// to blocks of at most 1,024 rows, so each set's rows end their runs together and every block
// holds the same mix of lengths. The block count follows round_block_count: the fewest full
// blocks, or one block per compute unit when those would leave CUs idle. In each block the sets go, heaviest first, to the least-loaded of
// the 16 waves with a layer left (rank_slot), which is how the part walk balances the waves
// it synchronizes at every part. For gene part p and layer (wave w, layer l) the 8 rows' runs in
// the part are r_0 .. r_7; the layer gets ceil(max r_g / 16) fills of 128 entries, entry k of
// group g's run at fill k / 16, slot g * 16 + k % 16; unused slots hold the pad gene (the zero
// weight row, value 0; of the parity opposite to the paired group's entry at that step).
// Each group's run is stored even genes first in even groups and odd genes first in odd
// groups (the LDS bank half of a weight row is its gene's parity). Fills are stored in
// (block, wave, part, layer) order: a wave's fills are one contiguous run across all parts,
// so the walk's fill prefetch continues through the part boundaries.
//
// Building: sort the rows by tail length, plan (block rows, slot rows and each layer's fill
// count and last step count), an exclusive scan of the counts into the fill index, then the
// fill. The plan
// and the fill walk each row the same way (a run is the entries from the cursor while the
// gene is below the part's end), so a fill never exceeds its plan; a row whose genes are not
// non-decreasing within [head, cols) -- which the columns-sorted flag promised -- is reported
// instead.
#include "qcsr_common.hpp"

#include <algorithm>
#include <cstdlib>

namespace cx {
namespace {

constexpr int kPlanChunk = 32;  // parts counted per pass of the plan kernel (LDS: 64 KB of runs)
constexpr std::uint32_t kNoSlotRow = 0xffffffffu;
constexpr std::uint32_t kLengthKeyBits = 24;  // tail lengths are sorted on 24 bits (longer ones tie)

struct PlanArgs {
    const std::int32_t *row_ptr;
    const std::int32_t *col_idx;
    const std::int32_t *head_end;
    const std::uint32_t *order;   // [rows]: rows by tail length, descending (ties by row)
    std::uint32_t rows;
    std::uint32_t cols;
    std::uint32_t first_part;
    std::uint32_t parts;          // parts in the stream
    std::uint32_t *slot_rows;     // [blocks][kStreamRows]
    std::uint32_t *counts;        // [blocks * kStreamWaves * parts * kStreamLayers + 1], (block, wave, part,
                                  // layer) order: fills per layer and part (last: 0)
    std::uint8_t *lasts;          // same order: step count of the last fill (0: none)
    std::uint32_t *error;         // [0]: a row not sorted within [head, cols); [1]: a block's fills reach 4 GiB
};

// Position of (block, wave, part, layer) in the fill index: a wave's layers of all parts
// are consecutive.
__device__ __forceinline__ std::uint64_t index_pos(std::uint32_t block, int wave, std::uint32_t part,
                                                   std::uint32_t parts, int layer) {
    return ((static_cast<std::uint64_t>(block) * kStreamWaves + wave) * parts + part) * kStreamLayers + layer;
}

// Sort keys of the rows: 2^24 - 1 - tail length (saturated), so an ascending stable sort gives
// descending lengths, ties by row.
__global__ __launch_bounds__(256) void tail_length_keys_kernel(const std::int32_t *row_ptr, const std::int32_t *head_end,
                                                               std::uint32_t rows, std::uint32_t *keys,
                                                               std::uint32_t *ids) {
    const std::uint32_t r = blockIdx.x * 256u + threadIdx.x;
    if (r >= rows) return;
    const std::int64_t len = static_cast<std::int64_t>(row_ptr[r + 1]) - head_end[r];
    constexpr std::int64_t kMax = (std::int64_t{1} << kLengthKeyBits) - 1;
    keys[r] = static_cast<std::uint32_t>(kMax - (len < 0 ? 0 : (len > kMax ? kMax : len)));
    ids[r] = r;
}

// The block's rows and the row of every slot. The sorted order is cut into sets of 8
// consecutive rows (nearly equal tail lengths, so a layer's 8 runs end together), dealt
// round-robin to the blocks (set S -> block S % blocks, local set S / blocks): every block
// holds the same mix of lengths. Inside the block the rows are ranked by tail length (ties by
// local position), ranks 8s .. 8s + 7 form set s, and the sets go, heaviest first, to the
// least-loaded wave with a layer left (ties: the lower wave), each wave's layers in the order
// its sets arrive, so the waves carry about equal work into every part barrier.
struct RankShared {
    int len[kStreamRows];             // tail length by local position (-1: empty)
    int by_rank[kStreamRows];         // tail length by rank
    int set_slot[kStreamSlots];       // wave * kStreamLayers + layer of set s
    std::uint32_t slot_row[kStreamRows];
    long long wave_load[kStreamWaves];
    int wave_used[kStreamWaves];
};

__device__ __forceinline__ std::uint32_t rank_slot(RankShared &r, const PlanArgs &a, std::uint32_t block,
                                                   std::uint32_t blocks, int tid) {
    const std::uint64_t at = (static_cast<std::uint64_t>(tid / 8) * blocks + block) * 8u + static_cast<std::uint64_t>(tid % 8);
    const std::uint32_t row = at < a.rows ? a.order[at] : a.rows;
    r.len[tid] = row < a.rows ? a.row_ptr[row + 1] - a.head_end[row] : -1;
    __syncthreads();
    const int my = r.len[tid];
    int rank = 0;
    for (int u = 0; u < kStreamRows; ++u) {
        const int v = r.len[u];
        rank += v > my || (v == my && u < tid) ? 1 : 0;
    }
    r.by_rank[rank] = my;
    __syncthreads();
    if (tid == 0) {
        for (int w = 0; w < kStreamWaves; ++w) {
            r.wave_load[w] = 0;
            r.wave_used[w] = 0;
        }
        for (int s = 0; s < kStreamSlots; ++s) {  // set loads are non-increasing in s
            long long load = 0;
            for (int k = 0; k < 8; ++k) load += r.by_rank[s * 8 + k] > 0 ? r.by_rank[s * 8 + k] : 0;
            int best = -1;
            for (int w = 0; w < kStreamWaves; ++w)
                if (r.wave_used[w] < kStreamLayers && (best < 0 || r.wave_load[w] < r.wave_load[best])) best = w;
            r.set_slot[s] = best * kStreamLayers + r.wave_used[best];
            ++r.wave_used[best];
            r.wave_load[best] += load;
        }
    }
    __syncthreads();
    r.slot_row[r.set_slot[rank / 8] * 8 + rank % 8] = row < a.rows ? row : kNoSlotRow;
    __syncthreads();
    return r.slot_row[tid];  // thread tid now works for slot tid
}

static_assert(sizeof(RankShared) + sizeof(std::uint16_t) * kPlanChunk * kStreamRows + sizeof(std::int64_t) * kStreamRows
                  <= 160u * 1024u,
              "the stream plan kernel's LDS exceeds gfx950's 160 KB");

// After the ranking, wave w counts the runs of its 64 slots (stream wave w) one row at a time:
// the row's tail is read 64 entries at a time, coalesced, each entry's part (within a window
// of kPlanChunk parts) comes from its gene, and the first lane of each part's segment adds the
// segment's size to the part's run. A row is reported (error word 0) when its genes go back to
// an earlier part, fall below the window, or reach cols or past it (entries left at the end).
__global__ __launch_bounds__(kStreamRows) void stream_plan_kernel(PlanArgs a) {
    __shared__ RankShared rs;
    __shared__ std::uint16_t runs[kPlanChunk][kStreamRows];
    __shared__ std::int64_t cursor[kStreamRows];
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const std::uint32_t block = blockIdx.x;
    const std::uint32_t row = rank_slot(rs, a, block, gridDim.x, tid);
    a.slot_rows[static_cast<std::uint64_t>(block) * kStreamRows + tid] = row;
    cursor[tid] = row != kNoSlotRow ? a.head_end[row] : 0;
    const std::uint64_t below = (std::uint64_t{1} << lane) - 1u;
    bool bad = false;  // per wave (lane 0 reports)
    for (std::uint32_t c0 = 0; c0 < a.parts; c0 += kPlanChunk) {
        const std::uint32_t cn = min(static_cast<std::uint32_t>(kPlanChunk), a.parts - c0);
        const std::int64_t lo = static_cast<std::int64_t>(a.first_part + c0) * kStreamPartGenes;
        for (int t = tid; t < kPlanChunk * kStreamRows; t += kStreamRows) (&runs[0][0])[t] = 0;
        __syncthreads();
        for (int sl = 0; sl < kWave; ++sl) {
            const int slot = wave * kWave + sl;
            const std::uint32_t r = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(rs.slot_row[slot])));
            if (r == kNoSlotRow || r >= a.rows) continue;
            const std::int64_t end = __builtin_amdgcn_readfirstlane(a.row_ptr[r + 1]);
            std::int64_t cur = cursor[slot];
            std::int64_t prev_pp = 0;  // part of the last entry taken
            while (cur < end) {
                const std::int64_t e = cur + lane;
                const bool valid = e < end;
                const std::int64_t gene = valid ? static_cast<std::int64_t>(a.col_idx[e]) : 0;
                const std::int64_t rel = gene - lo;
                const std::int64_t pp = rel >= 0 ? rel >> 10 : -1;
                const bool in = valid && pp >= 0 && pp < static_cast<std::int64_t>(cn);
                std::int64_t before = static_cast<std::int64_t>(__shfl_up(static_cast<int>(pp), 1, kWave));
                if (lane == 0) before = prev_pp;
                const std::uint64_t inb = __builtin_amdgcn_ballot_w64(in);
                const int n = __popcll(inb);
                // the window's entries must be a prefix, in non-decreasing parts, none below it
                const bool wrong = (in && pp < before) || (valid && rel < 0);
                if (__builtin_amdgcn_ballot_w64(wrong) != 0u || inb != (n == kWave ? ~std::uint64_t{0} : (std::uint64_t{1} << n) - 1u))
                    bad = true;
                const std::uint64_t heads = __builtin_amdgcn_ballot_w64(in && (lane == 0 || before != pp));
                if (in && ((heads >> lane) & 1u) != 0u) {
                    const std::uint64_t after = heads & ~(below | (std::uint64_t{1} << lane));
                    const std::uint64_t stop = after != 0u ? (after & (~after + 1u)) - 1u : ~std::uint64_t{0};
                    const int len = __popcll(inb & stop & ~below);
                    const int total = static_cast<int>(runs[pp][slot]) + len;
                    if (total > 0xffff) bad = true;
                    runs[pp][slot] = static_cast<std::uint16_t>(min(total, 0xffff));
                }
                if (n > 0) prev_pp = __builtin_amdgcn_readlane(static_cast<int>(pp), n - 1);
                cur += n;
                if (n < kWave) break;
            }
            if (lane == 0) cursor[slot] = cur;
        }
        __syncthreads();
        // one (part, wave, layer) per thread-iteration: the largest run of its 8 groups
        for (int t = tid; t < static_cast<int>(cn) * kStreamSlots; t += kStreamRows) {
            const int c = t / kStreamSlots, sl = t % kStreamSlots;
            int m = 0;
#pragma unroll
            for (int g = 0; g < 8; ++g) m = max(m, static_cast<int>(runs[c][sl * 8 + g]));
            const std::uint64_t k = index_pos(block, sl / kStreamLayers, c0 + c, a.parts, sl % kStreamLayers);
            const int fills = (m + 15) / 16;
            a.counts[k] = static_cast<std::uint32_t>(fills);
            a.lasts[k] = static_cast<std::uint8_t>(fills == 0 ? 0 : m - 16 * (fills - 1));
        }
        __syncthreads();
    }
    // genes at or past cols, or a walk stopped early: entries left over
    if (row != kNoSlotRow && cursor[tid] != a.row_ptr[row + 1]) bad = true;
    if (__builtin_amdgcn_ballot_w64(bad) != 0u && lane == 0) atomicOr(&a.error[0], 1u);
}

// index[k] = first fill | (last steps - 1) << 28; the scan left the first fills in index.
// The walk addresses a block's fills by 32-bit byte offsets: a block needing 2^32 bytes or
// more of fills is reported (error word 1).
__global__ __launch_bounds__(256) void stream_pack_kernel(std::uint32_t *index, const std::uint8_t *lasts,
                                                          std::uint64_t n, std::uint64_t per_block,
                                                          std::uint32_t max_block_fills, std::uint32_t *error) {
    const std::uint64_t k = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= n) return;
    const std::uint32_t first = index[k] & kFillMask;
    if (k % per_block == 0u && (index[k + per_block] & kFillMask) - first >= max_block_fills) atomicOr(&error[1], 1u);
    if (lasts[k] != 0u) index[k] = first | static_cast<std::uint32_t>(lasts[k] - 1u) << 28;
}

__global__ __launch_bounds__(256) void fill_pattern_kernel(std::uint32_t *p, std::uint64_t words, std::uint32_t v) {
    for (std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words;
         i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x)
        p[i] = v;
}

struct FillArgs {
    const std::int32_t *row_ptr;
    const std::int32_t *packed_row_ptr;
    const std::int32_t *col_idx;
    const std::uint8_t *packed;
    const std::int32_t *head_end;
    const std::uint32_t *slot_rows;
    const std::uint32_t *index;
    void *entries;
    std::uint32_t cols;
    std::uint32_t first_part;
    std::uint32_t parts;
};

// One wave per slot, the 64 slots of stream wave w taken in turn by the workgroup's wave w.
// The row's tail is read 64 entries at a time, coalesced (a thread per row read 64 unrelated
// rows per load and missed the caches on most of them). Columns are sorted, so the entries of
// one gene part are consecutive lanes: ballots find each part's segment, and an entry's slot
// in its part's run is its rank among the segment's entries of its parity class plus the
// counts of earlier chunks (LDS, per part); entries of the other parity follow all the
// preferred ones, whose total per part a first pass counts. Parts are handled 64 at a time.
// Every write is bounded by the fills the plan gave the layer, so a row the plan reported as
// unsorted cannot write past them.
template<int kBits>
__global__ __launch_bounds__(kStreamRows) void stream_fill_kernel(FillArgs a) {
    constexpr bool kWide = kBits == 8;
    constexpr std::uint32_t kMask = (1u << kBits) - 1u;
    __shared__ std::uint32_t part_counts[kStreamWaves][3][kWave];  // per wave and window part: preferred total, carries
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const std::uint32_t block = blockIdx.x;
    std::uint32_t *npref = part_counts[wave][0], *cpref = part_counts[wave][1], *coth = part_counts[wave][2];
    const std::uint64_t below = (std::uint64_t{1} << lane) - 1u;  // lanes before this one
    auto lds_order = [] { __asm__ volatile("" ::: "memory"); };
    for (int s = 0; s < 64; ++s) {
        const int slot = wave * 64 + s;
        const std::uint32_t row = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(
            static_cast<int>(a.slot_rows[static_cast<std::uint64_t>(block) * kStreamRows + slot])));
        if (row == kNoSlotRow) continue;
        const int layer = (slot / 8) % kStreamLayers, g = slot % 8;
        const std::uint32_t pref = static_cast<std::uint32_t>(g & 1);  // parity stored first
        const std::int64_t rb = __builtin_amdgcn_readfirstlane(a.row_ptr[row]);
        const std::int64_t end = __builtin_amdgcn_readfirstlane(a.row_ptr[row + 1]);
        const std::int64_t pbit = static_cast<std::int64_t>(__builtin_amdgcn_readfirstlane(a.packed_row_ptr[row])) * 8;
        std::int64_t hs = __builtin_amdgcn_readfirstlane(a.head_end[row]);
        for (std::uint32_t p0 = 0; p0 < a.parts && hs < end; p0 += kWave) {
            const std::int64_t lo = static_cast<std::int64_t>(a.first_part + p0) * kStreamPartGenes;
            const std::uint32_t window = min(static_cast<std::uint32_t>(kWave), a.parts - p0);
            lds_order();
            npref[lane] = 0u;
            cpref[lane] = 0u;
            coth[lane] = 0u;
            lds_order();
            // An entry of the window: its part (relative to p0) and parity class; segment heads
            // are the first lane of each part's run in the chunk.
            struct Lane {
                bool in, pref;
                std::uint32_t pp, local;
                std::uint64_t heads;
            };
            auto classify = [&](std::int64_t e, std::int64_t limit) {
                Lane L{};
                const std::int64_t gene = e < limit ? static_cast<std::int64_t>(a.col_idx[e]) : -1;
                const std::int64_t rel = gene - lo;
                L.in = e < limit && rel >= 0 && (rel >> 10) < static_cast<std::int64_t>(window);
                L.pp = L.in ? static_cast<std::uint32_t>(rel >> 10) : 0u;
                L.local = static_cast<std::uint32_t>(rel & (kStreamPartGenes - 1));
                L.pref = L.in && (L.local & 1u) == pref;
                const std::uint32_t prev_pp = static_cast<std::uint32_t>(__shfl_up(static_cast<int>(L.pp), 1, kWave));
                const std::uint64_t inb = __builtin_amdgcn_ballot_w64(L.in);
                const bool prev_in = lane > 0 && ((inb >> (lane - 1)) & 1u) != 0u;
                L.heads = __builtin_amdgcn_ballot_w64(L.in && (!prev_in || prev_pp != L.pp));
                return L;
            };
            // lanes of this lane's segment: from its head up to (not including) the next head
            auto segment = [&](const Lane &L, std::uint64_t inb) {
                const std::uint64_t upto = L.heads & (below | (std::uint64_t{1} << lane));
                const int head = upto != 0u ? 63 - __builtin_clzll(upto) : 0;
                const std::uint64_t after = L.heads & ~(below | (std::uint64_t{1} << lane));
                const std::uint64_t stop = after != 0u ? (after & (~after + 1u)) - 1u : ~std::uint64_t{0};
                return inb & stop & ~((std::uint64_t{1} << head) - 1u);
            };
            // pass 1: preferred entries per part, and the end of the window's entries
            std::int64_t he = hs;
            for (std::int64_t e0 = hs; e0 < end; e0 += kWave) {
                const Lane L = classify(e0 + lane, end);
                const std::uint64_t inb = __builtin_amdgcn_ballot_w64(L.in);
                const std::uint64_t pb = __builtin_amdgcn_ballot_w64(L.pref);
                if (L.in && ((L.heads >> lane) & 1u) != 0u) npref[L.pp] += static_cast<std::uint32_t>(__popcll(pb & segment(L, inb)));
                lds_order();
                const int n = __popcll(inb);  // sorted rows: the window's entries are a prefix
                he = e0 + n;
                if (n < kWave) break;
            }
            // pass 2: each entry's slot in its part's run, and its write
            for (std::int64_t e0 = hs; e0 < he; e0 += kWave) {
                const std::int64_t e = e0 + lane;
                const Lane L = classify(e, he);
                const std::uint64_t inb = __builtin_amdgcn_ballot_w64(L.in);
                const std::uint64_t pb = __builtin_amdgcn_ballot_w64(L.pref);
                const std::uint64_t ob = inb & ~pb;
                const std::uint64_t seg = segment(L, inb);
                const std::uint64_t before = seg & below;
                std::uint32_t k = 0u;
                if (L.in)
                    k = L.pref ? cpref[L.pp] + static_cast<std::uint32_t>(__popcll(pb & before))
                               : npref[L.pp] + coth[L.pp] + static_cast<std::uint32_t>(__popcll(ob & before));
                lds_order();
                if (L.in) {
                    const std::uint64_t ix = index_pos(block, wave, p0 + L.pp, a.parts, layer);
                    const std::uint32_t fill0 = a.index[ix] & kFillMask;
                    const std::uint32_t fills = (a.index[ix + 1u] & kFillMask) - fill0;
                    if (k / 16u < fills) {
                        const std::int64_t bit = pbit + (e - rb) * kBits;
                        const std::uint32_t code = (static_cast<std::uint32_t>(a.packed[bit >> 3]) >> (bit & 7)) & kMask;
                        const std::uint64_t pos = static_cast<std::uint64_t>(fill0 + k / 16u) * 128u + g * 16u + k % 16u;
                        if constexpr (kWide) static_cast<std::uint32_t *>(a.entries)[pos] = L.local | code << 16;
                        else static_cast<std::uint16_t *>(a.entries)[pos] = static_cast<std::uint16_t>(L.local | code << 11);
                    }
                    if (((L.heads >> lane) & 1u) != 0u) {
                        cpref[L.pp] += static_cast<std::uint32_t>(__popcll(pb & seg));
                        coth[L.pp] += static_cast<std::uint32_t>(__popcll(ob & seg));
                    }
                }
                lds_order();
            }
            hs = he;
        }
    }
}

// Pads of a fill take the parity opposite to the paired group's entry at the same step
// (groups 2i and 2i + 1 read in the same LDS cycle; a weight row of gene g occupies bank
// half g & 1): one thread per (fill, group pair, step).
template<bool kWide>
__global__ __launch_bounds__(256) void stream_pad_parity_kernel(void *entries, std::uint64_t fills) {
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= fills * 64u) return;
    const std::uint64_t fill = i / 64u;
    const std::uint32_t pair = static_cast<std::uint32_t>(i % 64u) / 16u, step = static_cast<std::uint32_t>(i % 16u);
    const std::uint64_t e0 = fill * 128u + (2u * pair) * 16u + step, e1 = e0 + 16u;
    constexpr std::uint32_t kGeneMask = kWide ? 0xffffu : 0x7ffu;
    auto get = [&](std::uint64_t e) -> std::uint32_t {
        return kWide ? static_cast<std::uint32_t *>(entries)[e] : static_cast<std::uint16_t *>(entries)[e];
    };
    auto put = [&](std::uint64_t e, std::uint32_t v) {
        if constexpr (kWide) static_cast<std::uint32_t *>(entries)[e] = v;
        else static_cast<std::uint16_t *>(entries)[e] = static_cast<std::uint16_t>(v);
    };
    const std::uint32_t a = get(e0), b = get(e1);
    const bool pa = (a & kGeneMask) >= kStreamPad, pb = (b & kGeneMask) >= kStreamPad;
    if (pa && !pb) put(e0, (b & 1u) != 0u ? kStreamPad : kStreamPadOdd);
    if (pb && !pa) put(e1, (a & 1u) != 0u ? kStreamPad : kStreamPadOdd);
}

constexpr std::uint64_t align256(std::uint64_t b) { return (b + 255u) & ~std::uint64_t{255u}; }

struct PlanSizes {
    std::uint64_t n;  // fill-index entries before the sentinel
    std::uint64_t error, slot_rows, index, counts, lasts, scan, rows4, sort, total;
    std::uint32_t blocks, parts;
};

PlanSizes plan_sizes(const cx_qcsr_matrix *m, const cx_qcsr_hybrid_layout *L) {
    PlanSizes s{};
    s.blocks = round_block_count(m->rows, kStreamRows, blocks_per_round(), false);
    const std::uint32_t all_parts = (m->cols + kStreamPartGenes - 1) / kStreamPartGenes;
    const std::uint32_t first = L->head_cols / kStreamPartGenes;
    s.parts = all_parts > first ? all_parts - first : 0u;
    s.n = static_cast<std::uint64_t>(s.blocks) * s.parts * kStreamSlots;
    s.error = 256;
    s.slot_rows = align256(static_cast<std::uint64_t>(s.blocks) * kStreamRows * 4u);
    s.index = align256((s.n + 1u) * 4u);
    s.counts = align256((s.n + 1u) * 4u);
    s.lasts = align256(s.n + 1u);
    s.scan = align256(scan_workspace_bytes(s.n + 1u));
    s.rows4 = align256(static_cast<std::uint64_t>(m->rows) * 4u);  // keys, ids, sorted keys, order
    s.sort = align256(sort_pairs_workspace_bytes(m->rows, kLengthKeyBits));
    s.total = s.error + s.slot_rows + s.index + s.counts + s.lasts + s.scan + 4u * s.rows4 + s.sort;
    return s;
}

int validate_stream(const cx_qcsr_matrix *m, const cx_qcsr_hybrid_layout *L, const char *who) {
    if (m == nullptr || L == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, who);
    if (m->bits != 1u && m->bits != 2u && m->bits != 4u && m->bits != 8u)
        return fail(CX_STATUS_UNSUPPORTED, "quantized CSR tail stream: codes of 1, 2, 4 or 8 bits only");
    if ((m->flags & CX_QCSR_COLUMNS_SORTED) == 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "quantized CSR tail stream: rows must be sorted (CX_QCSR_COLUMNS_SORTED)");
    if (L->rows != m->rows || L->bits != m->bits || L->nnz != m->nnz || L->head_end == nullptr
        || L->head_cols % kStreamPartGenes != 0u || L->head_cols > m->cols)
        return fail(CX_STATUS_INVALID_ARGUMENT, "quantized CSR tail stream: the hybrid layout was not prepared for this matrix");
    if (m->rows == 0u || m->cols == 0u)
        return fail(CX_STATUS_INVALID_SHAPE, "quantized CSR tail stream: empty matrix");
    if (m->row_ptr == nullptr || m->packed_row_ptr == nullptr
        || (m->nnz != 0u && (m->col_idx == nullptr || m->packed_values == nullptr)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "quantized CSR tail stream: null structure or codes");
    const PlanSizes s = plan_sizes(m, L);
    if (s.n + 1u > 0x7fffffffull)
        return fail(CX_STATUS_INVALID_SHAPE, "quantized CSR tail stream: too many (block, part, layer) entries");
    return CX_STATUS_SUCCESS;
}

} // namespace

std::uint32_t blocks_per_round() {
    if (const char *env = std::getenv("CX_BLOCKS_PER_ROUND")) {
        char *end = nullptr;
        const unsigned long v = std::strtoul(env, &end, 10);
        if (end != env && *end == '\0' && v > 0ul && v <= 0xffffffffull) return static_cast<std::uint32_t>(v);
    }
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess
        || cus < 0) {
        (void)hipGetLastError();
        return 0u;
    }
    return static_cast<std::uint32_t>(cus);
}

} // namespace cx

extern "C" int cx_qcsr_tail_plan_bytes(const cx_qcsr_matrix *m, const cx_qcsr_hybrid_layout *layout, uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (bytes == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_tail_plan_bytes: null bytes");
    const int rc = validate_stream(m, layout, "cx_qcsr_tail_plan_bytes: null argument");
    if (rc != CX_STATUS_SUCCESS) return rc;
    *bytes = plan_sizes(m, layout).total;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_tail_plan(const cx_qcsr_matrix *m, const cx_qcsr_hybrid_layout *layout, void *storage,
                                 uint64_t storage_bytes, cx_qcsr_tail_stream *out, uint64_t *entry_bytes,
                                 void *stream) {
    using namespace cx;
    clear_error();
    int rc = validate_stream(m, layout, "cx_qcsr_tail_plan: null argument");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (out == nullptr || entry_bytes == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_tail_plan: null output");
    const PlanSizes sz = plan_sizes(m, layout);
    if (storage == nullptr || storage_bytes < sz.total || (reinterpret_cast<std::uintptr_t>(storage) & 255u) != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_tail_plan: storage must be 256-byte aligned and hold cx_qcsr_tail_plan_bytes");
    auto *base = static_cast<unsigned char *>(storage);
    auto *error = reinterpret_cast<std::uint32_t *>(base);
    std::uint64_t off = sz.error;
    auto *slot_rows = reinterpret_cast<std::uint32_t *>(base + off);
    off += sz.slot_rows;
    auto *index = reinterpret_cast<std::uint32_t *>(base + off);
    off += sz.index;
    auto *counts = reinterpret_cast<std::uint32_t *>(base + off);
    off += sz.counts;
    auto *lasts = reinterpret_cast<std::uint8_t *>(base + off);
    off += sz.lasts;
    void *scan_ws = base + off;
    off += sz.scan;
    auto *keys = reinterpret_cast<std::uint32_t *>(base + off);
    auto *ids = reinterpret_cast<std::uint32_t *>(base + off + sz.rows4);
    auto *keys_sorted = reinterpret_cast<std::uint32_t *>(base + off + 2u * sz.rows4);
    auto *order = reinterpret_cast<std::uint32_t *>(base + off + 3u * sz.rows4);
    void *sort_ws = base + off + 4u * sz.rows4;

    const hipStream_t s = static_cast<hipStream_t>(stream);
    // rows by tail length over the whole matrix: blocks of similar rows, the longest first
    hipLaunchKernelGGL(tail_length_keys_kernel, dim3((m->rows + 255u) / 256u), dim3(256), 0, s, m->row_ptr,
                       layout->head_end, m->rows, keys, ids);
    rc = check_launch("cx_qcsr_tail_plan");
    if (rc != CX_STATUS_SUCCESS) return rc;
    rc = sort_pairs(keys, ids, keys_sorted, order, m->rows, kLengthKeyBits, sort_ws, sz.sort, s);
    if (rc != CX_STATUS_SUCCESS) return rc;
    // error words, and the sentinel count that the scan turns into the total
    hipLaunchKernelGGL(fill_pattern_kernel, dim3(1), dim3(64), 0, s, error, std::uint64_t{4}, 0u);
    hipLaunchKernelGGL(fill_pattern_kernel, dim3(1), dim3(64), 0, s, counts + sz.n, std::uint64_t{1}, 0u);
    PlanArgs pa{};
    pa.row_ptr = m->row_ptr;
    pa.col_idx = m->col_idx;
    pa.head_end = layout->head_end;
    pa.order = order;
    pa.rows = m->rows;
    pa.cols = m->cols;
    pa.first_part = layout->head_cols / kStreamPartGenes;
    pa.parts = sz.parts;
    pa.slot_rows = slot_rows;
    pa.counts = counts;
    pa.lasts = lasts;
    pa.error = error;
    hipLaunchKernelGGL(stream_plan_kernel, dim3(sz.blocks), dim3(kStreamRows), 0, s, pa);
    rc = check_launch("cx_qcsr_tail_plan");
    if (rc != CX_STATUS_SUCCESS) return rc;
    rc = exclusive_scan_u32(counts, index, sz.n + 1u, scan_ws, s);
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (sz.n != 0u) {
        const std::uint32_t max_block_fills = m->bits == 8u ? (1u << 23) - 4u : (1u << 24) - 4u;
        hipLaunchKernelGGL(stream_pack_kernel, dim3(static_cast<unsigned>((sz.n + 255u) / 256u)), dim3(256), 0, s,
                           index, lasts, sz.n, static_cast<std::uint64_t>(sz.parts) * kStreamSlots, max_block_fills,
                           error);
        rc = check_launch("cx_qcsr_tail_plan");
        if (rc != CX_STATUS_SUCCESS) return rc;
    }
    std::uint32_t host[2] = {0u, 0u};
    std::uint32_t total = 0u;
    hipError_t e = hipMemcpyAsync(host, error, sizeof(host), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipMemcpyAsync(&total, index + sz.n, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "cx_qcsr_tail_plan");
    if (host[0] != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_tail_plan: a row's genes are not sorted within [head_cols, cols) despite CX_QCSR_COLUMNS_SORTED");
    // The u32 scan is exact: a layer's fills are at most its largest run / 16 + 1, so the
    // total is below nnz / 16 + n < 2^32 (nnz and n are below 2^31).
    if (host[1] != 0u)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_tail_plan: a block needs 4 GiB of stream or more");
    if (total >= kFillMask)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_tail_plan: the stream needs 2^28 fills or more");
    const std::uint64_t fill_bytes = m->bits == 8u ? 512u : 256u;
    cx_qcsr_tail_stream t{};
    t.rows = m->rows;
    t.first_part = layout->head_cols / kStreamPartGenes;
    t.parts = sz.parts;
    t.blocks = sz.blocks;
    t.block_rows = kStreamRows;
    t.layers = kStreamLayers;
    t.bits = m->bits;
    t.entry_bytes = m->bits == 8u ? 4u : 2u;
    t.fills = total;
    t.nnz = m->nnz;
    t.slot_rows = slot_rows;
    t.fill_index = index;
    t.entries = nullptr;
    *out = t;
    // three fills of slack: the walk's prefetch reads up to three fills past a block's last
    *entry_bytes = (static_cast<std::uint64_t>(total) + 3u) * fill_bytes;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_tail_fill(const cx_qcsr_matrix *m, const cx_qcsr_hybrid_layout *layout,
                                 cx_qcsr_tail_stream *ts, void *entries, uint64_t entry_bytes, void *stream) {
    using namespace cx;
    clear_error();
    int rc = validate_stream(m, layout, "cx_qcsr_tail_fill: null argument");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (ts == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_tail_fill: null stream");
    const PlanSizes sz = plan_sizes(m, layout);
    const std::uint64_t fill_bytes = m->bits == 8u ? 512u : 256u;
    if (ts->rows != m->rows || ts->bits != m->bits || ts->nnz != m->nnz || ts->parts != sz.parts
        || ts->blocks != sz.blocks || ts->block_rows != kStreamRows || ts->layers != kStreamLayers
        || ts->first_part != layout->head_cols / kStreamPartGenes
        || ts->slot_rows == nullptr || ts->fill_index == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_tail_fill: the stream was not planned for this matrix");
    const std::uint64_t need = (ts->fills + 3u) * fill_bytes;
    if (entries == nullptr || entry_bytes < need || (reinterpret_cast<std::uintptr_t>(entries) & 255u) != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_tail_fill: entries must be 256-byte aligned and hold the bytes cx_qcsr_tail_plan returned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const std::uint32_t pad = m->bits == 8u ? kStreamPad : (kStreamPad | kStreamPad << 16);
    const std::uint64_t words = need / 4u;
    hipLaunchKernelGGL(fill_pattern_kernel, dim3(static_cast<unsigned>(std::min<std::uint64_t>((words + 255u) / 256u, 65536u))),
                       dim3(256), 0, s, static_cast<std::uint32_t *>(entries), words, pad);
    FillArgs fa{};
    fa.row_ptr = m->row_ptr;
    fa.packed_row_ptr = m->packed_row_ptr;
    fa.col_idx = m->col_idx;
    fa.packed = m->packed_values;
    fa.head_end = layout->head_end;
    fa.slot_rows = ts->slot_rows;
    fa.index = ts->fill_index;
    fa.entries = entries;
    fa.cols = m->cols;
    fa.first_part = ts->first_part;
    fa.parts = ts->parts;
    const dim3 grid(sz.blocks), block(kStreamRows);
    switch (m->bits) {
    case 1: hipLaunchKernelGGL(stream_fill_kernel<1>, grid, block, 0, s, fa); break;
    case 2: hipLaunchKernelGGL(stream_fill_kernel<2>, grid, block, 0, s, fa); break;
    case 4: hipLaunchKernelGGL(stream_fill_kernel<4>, grid, block, 0, s, fa); break;
    default: hipLaunchKernelGGL(stream_fill_kernel<8>, grid, block, 0, s, fa); break;
    }
    rc = check_launch("cx_qcsr_tail_fill");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (ts->fills != 0u) {
        const std::uint64_t threads = ts->fills * 64u;
        const dim3 pgrid(static_cast<unsigned>((threads + 255u) / 256u));
        if (m->bits == 8u) hipLaunchKernelGGL(stream_pad_parity_kernel<true>, pgrid, dim3(256), 0, s, entries, ts->fills);
        else hipLaunchKernelGGL(stream_pad_parity_kernel<false>, pgrid, dim3(256), 0, s, entries, ts->fills);
        rc = check_launch("cx_qcsr_tail_fill");
        if (rc != CX_STATUS_SUCCESS) return rc;
    }
    ts->entries = entries;
    return CX_STATUS_SUCCESS;
}
