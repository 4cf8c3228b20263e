// sort.hip -- stable LSD radix sort of (u32 key, u32 value) pairs and an exclusive u32 scan,
// the device primitives behind the transposed CSR structure (and any other one-time
// structure build that needs a counting sort).
//
// Radix pass (8-bit digit), per tile of kTileItems = 4096 pairs (256 threads, wave w owns
// items [1024 w, 1024 w + 1024) as 16 rounds of 64 consecutive items):
//   1. histogram: in each round the lanes holding equal digits find each other with eight
//      ballots (one per digit bit); the highest lane of each digit group adds the group's
//      size to its wave's LDS counter -- no atomics, no per-lane LDS traffic.
//      Counts go to hist[digit * tiles + tile] (digit-major).
//   2. exclusive scan of hist: offset of (digit, tile) in the output.
//   3. scatter: same ballots; the tile is first reordered in LDS by digit (wave bases per
//      digit = the digit's tile-local start + counts of the earlier waves; inside a wave the
//      rounds run in order, each lane's slot = base + running count of its digit + its rank
//      among the lower lanes of its group), then written out with consecutive threads on
//      consecutive slots of each digit's run (global slot = tile offset of the digit +
//      position in the run). The output order is the input order within equal digits, so
//      the sort is stable and deterministic.
// Keys are sorted on their low key_bits bits (passes = ceil(key_bits / 8)).
#include "cx_common.hpp"

namespace cx {
namespace {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kRounds = 16;
constexpr int kTileItems = kSortThreads * kRounds;  // 4096
constexpr int kScanItems = kSortThreads * 16;       // 4096 per scan block

__device__ __forceinline__ std::uint64_t lanemask_lt() {
    const std::uint32_t lane = __lane_id();
    return lane == 0 ? 0ull : (~0ull >> (64u - lane));
}

// Lanes of the wave (among `active`) holding the same 8-bit digit as this lane.
__device__ __forceinline__ std::uint64_t digit_peers(std::uint32_t digit, std::uint64_t active) {
    std::uint64_t peers = active;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const std::uint64_t set = __ballot((digit >> b) & 1u);
        peers &= ((digit >> b) & 1u) ? set : ~set;
    }
    return peers;
}

struct PassArgs {
    const std::uint32_t *keys_in;
    const std::uint32_t *vals_in;  // NULL: value = item index
    std::uint32_t *keys_out;
    std::uint32_t *vals_out;
    std::uint32_t *hist;           // 256 * tiles
    std::uint32_t count;
    std::uint32_t tiles;
    std::uint32_t shift;
};

__device__ __forceinline__ std::uint32_t item_index(std::uint32_t tile, int wave, int round,
                                                    int lane) {
    return tile * static_cast<std::uint32_t>(kTileItems) + static_cast<std::uint32_t>(wave) * 1024u
        + static_cast<std::uint32_t>(round) * 64u + static_cast<std::uint32_t>(lane);
}

__global__ __launch_bounds__(kSortThreads) void radix_histogram(PassArgs a) {
    __shared__ std::uint32_t counts[kSortWaves][256];
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t tile = blockIdx.x;
    for (int d = lane; d < 256; d += kWave) counts[wave][d] = 0u;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int r = 0; r < kRounds; ++r) {
        const std::uint32_t i = item_index(tile, wave, r, lane);
        const bool valid = i < a.count;
        const std::uint32_t digit = valid ? (a.keys_in[i] >> a.shift) & 255u : 0u;
        const std::uint64_t active = __ballot(valid);
        if (active == 0u) break;
        const std::uint64_t peers = digit_peers(digit, active);
        const std::uint64_t higher = peers & ~lanemask_lt() & ~(1ull << lane);
        if (valid && higher == 0u) counts[wave][digit] += static_cast<std::uint32_t>(__popcll(peers));
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    const int d = static_cast<int>(threadIdx.x);
    std::uint32_t total = 0u;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) total += counts[w][d];
    a.hist[static_cast<std::uint64_t>(d) * a.tiles + tile] = total;
}

__global__ __launch_bounds__(kSortThreads) void radix_scatter(PassArgs a) {
    __shared__ std::uint32_t counts[kSortWaves][256];
    __shared__ std::uint32_t base[kSortWaves][256];   // tile-local start of (wave, digit)
    __shared__ std::uint32_t delta[256];              // global minus tile-local position
    __shared__ std::uint32_t wave_sums[kSortWaves];
    __shared__ std::uint32_t sk[kTileItems], sv[kTileItems];
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t tile = blockIdx.x;

    std::uint32_t key[kRounds], val[kRounds], digit[kRounds];
    std::uint64_t peers[kRounds];
    for (int d = lane; d < 256; d += kWave) counts[wave][d] = 0u;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
        const std::uint32_t i = item_index(tile, wave, r, lane);
        const bool valid = i < a.count;
        key[r] = valid ? a.keys_in[i] : 0u;
        val[r] = valid ? (a.vals_in != nullptr ? a.vals_in[i] : i) : 0u;
        digit[r] = (key[r] >> a.shift) & 255u;
        const std::uint64_t active = __ballot(valid);
        peers[r] = digit_peers(digit[r], active);
        const std::uint64_t higher = peers[r] & ~lanemask_lt() & ~(1ull << lane);
        if (valid && higher == 0u) counts[wave][digit[r]] += static_cast<std::uint32_t>(__popcll(peers[r]));
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    {
        // per digit: the tile's count, its tile-local start (exclusive scan over digits, one
        // digit per thread), the waves' local starts, and the shift to the global output
        const int d = static_cast<int>(threadIdx.x);
        std::uint32_t total = 0u;
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) total += counts[w][d];
        std::uint32_t incl = total;  // inclusive scan inside the wave
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const std::uint32_t o = static_cast<std::uint32_t>(__shfl_up(static_cast<int>(incl), off, kWave));
            if (lane >= off) incl += o;
        }
        if (lane == kWave - 1) wave_sums[wave] = incl;
        __syncthreads();
        std::uint32_t start = incl - total;
        for (int w = 0; w < wave; ++w) start += wave_sums[w];
        delta[d] = a.hist[static_cast<std::uint64_t>(d) * a.tiles + tile] - start;
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) {
            base[w][d] = start;
            start += counts[w][d];
        }
    }
    __syncthreads();
    // tile-local stable order in LDS: wave, then round, then rank among equal digits
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
        const std::uint32_t i = item_index(tile, wave, r, lane);
        const bool valid = i < a.count;
        const std::uint64_t below = peers[r] & lanemask_lt();
        const std::uint32_t slot = base[wave][digit[r]] + static_cast<std::uint32_t>(__popcll(below));
        if (valid) {
            sk[slot] = key[r];
            sv[slot] = val[r];
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const std::uint64_t higher = peers[r] & ~lanemask_lt() & ~(1ull << lane);
        if (valid && higher == 0u) base[wave][digit[r]] += static_cast<std::uint32_t>(__popcll(peers[r]));
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    // equal digits are now contiguous: consecutive threads write consecutive output slots
    const std::uint32_t first = tile * static_cast<std::uint32_t>(kTileItems);
    const std::uint32_t n = a.count - first < static_cast<std::uint32_t>(kTileItems)
        ? a.count - first : static_cast<std::uint32_t>(kTileItems);
#pragma unroll 4
    for (std::uint32_t i = threadIdx.x; i < n; i += kSortThreads) {
        const std::uint32_t k = sk[i];
        const std::uint32_t slot = delta[(k >> a.shift) & 255u] + i;
        a.keys_out[slot] = k;
        a.vals_out[slot] = sv[i];
    }
}

// ---- exclusive scan (u32, wrap-around on overflow: callers bound the total) ----------

// Inclusive scan of one value per thread across the 256-thread block; returns the block
// total through `total`.
__device__ __forceinline__ std::uint32_t block_inclusive(std::uint32_t v, std::uint32_t *total) {
    __shared__ std::uint32_t wave_sums[kSortWaves];
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int wave = static_cast<int>(threadIdx.x) / kWave;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const std::uint32_t up = __shfl_up(v, o, kWave);
        if (lane >= o) v += up;
    }
    if (lane == kWave - 1) wave_sums[wave] = v;
    __syncthreads();
    std::uint32_t before = 0u, all = 0u;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) {
        const std::uint32_t s = wave_sums[w];
        before += w < wave ? s : 0u;
        all += s;
    }
    __syncthreads();
    *total = all;
    return v + before;
}

// Per block of kScanItems: its sum.
__global__ __launch_bounds__(kSortThreads) void scan_reduce(const std::uint32_t *in, std::uint64_t n,
                                                            std::uint32_t *block_sums) {
    const std::uint64_t begin = static_cast<std::uint64_t>(blockIdx.x) * kScanItems;
    std::uint32_t s = 0u;
    for (int k = 0; k < kScanItems / kSortThreads; ++k) {
        const std::uint64_t i = begin + static_cast<std::uint64_t>(k) * kSortThreads + threadIdx.x;
        if (i < n) s += in[i];
    }
    std::uint32_t total;
    block_inclusive(s, &total);
    if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// One block: exclusive scan of the block sums in place (sequential over chunks of 256).
__global__ __launch_bounds__(kSortThreads) void scan_block_sums(std::uint32_t *sums, std::uint32_t blocks) {
    std::uint32_t carry = 0u;
    for (std::uint32_t c0 = 0; c0 < blocks; c0 += kSortThreads) {
        const std::uint32_t i = c0 + threadIdx.x;
        const std::uint32_t v = i < blocks ? sums[i] : 0u;
        std::uint32_t total;
        const std::uint32_t inc = block_inclusive(v, &total);
        if (i < blocks) sums[i] = carry + inc - v;
        carry += total;
    }
}

// Exclusive scan of each block's items with the block's offset. Each thread owns 16
// consecutive items.
__global__ __launch_bounds__(kSortThreads) void scan_apply(const std::uint32_t *in, std::uint64_t n,
                                                           const std::uint32_t *block_offsets,
                                                           std::uint32_t *out) {
    constexpr int kPer = kScanItems / kSortThreads;
    const std::uint64_t begin = static_cast<std::uint64_t>(blockIdx.x) * kScanItems
        + static_cast<std::uint64_t>(threadIdx.x) * kPer;
    std::uint32_t v[kPer];
    std::uint32_t s = 0u;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        v[k] = begin + k < n ? in[begin + k] : 0u;
        s += v[k];
    }
    std::uint32_t total;
    std::uint32_t run = block_inclusive(s, &total) - s + block_offsets[blockIdx.x];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        if (begin + k < n) out[begin + k] = run;
        run += v[k];
    }
}

std::uint64_t align256(std::uint64_t b) { return (b + 255u) & ~static_cast<std::uint64_t>(255u); }

} // namespace

std::uint64_t scan_workspace_bytes(std::uint64_t n) {
    const std::uint64_t blocks = (n + kScanItems - 1) / kScanItems;
    return align256(blocks * 4u);
}

int exclusive_scan_u32(const std::uint32_t *in, std::uint32_t *out, std::uint64_t n, void *workspace,
                       hipStream_t stream) {
    if (n == 0u) return CX_STATUS_SUCCESS;
    const std::uint64_t blocks = (n + kScanItems - 1) / kScanItems;
    if (blocks > 0xFFFFFFFFull) return fail(CX_STATUS_INVALID_SHAPE, "scan: too many items");
    auto *sums = static_cast<std::uint32_t *>(workspace);
    const unsigned nb = static_cast<unsigned>(blocks);
    hipLaunchKernelGGL(scan_reduce, dim3(nb), dim3(kSortThreads), 0, stream, in, n, sums);
    hipLaunchKernelGGL(scan_block_sums, dim3(1), dim3(kSortThreads), 0, stream, sums, nb);
    hipLaunchKernelGGL(scan_apply, dim3(nb), dim3(kSortThreads), 0, stream, in, n, sums, out);
    return check_launch("exclusive_scan_u32");
}

std::uint64_t sort_pairs_workspace_bytes(std::uint64_t count, std::uint32_t key_bits) {
    const std::uint32_t passes = (key_bits + 7u) / 8u;
    const std::uint64_t tiles = (count + kTileItems - 1) / kTileItems;
    const std::uint64_t hist = tiles * 256u;
    std::uint64_t bytes = 2u * align256(hist * 4u) + scan_workspace_bytes(hist);
    if (passes >= 2u) bytes += 2u * align256(count * 4u);  // ping-pong pair
    return bytes;
}

int sort_pairs(const std::uint32_t *keys_in, const std::uint32_t *vals_in, std::uint32_t *keys_out,
               std::uint32_t *vals_out, std::uint64_t count, std::uint32_t key_bits,
               void *workspace, std::uint64_t workspace_bytes, hipStream_t stream) {
    if (key_bits == 0u || key_bits > 32u) return fail(CX_STATUS_INVALID_SHAPE, "sort: key_bits must be 1..32");
    if (count > 0xFFFFFFFFull - kTileItems) return fail(CX_STATUS_INVALID_SHAPE, "sort: count exceeds u32 indexing");
    if (workspace_bytes < sort_pairs_workspace_bytes(count, key_bits))
        return fail(CX_STATUS_INVALID_ARGUMENT, "sort: workspace too small");
    if (count == 0u) return CX_STATUS_SUCCESS;
    const std::uint32_t passes = (key_bits + 7u) / 8u;
    const std::uint32_t tiles = static_cast<std::uint32_t>((count + kTileItems - 1) / kTileItems);
    const std::uint64_t hist_n = static_cast<std::uint64_t>(tiles) * 256u;
    auto *ws = static_cast<unsigned char *>(workspace);
    auto *hist = reinterpret_cast<std::uint32_t *>(ws);
    ws += align256(hist_n * 4u);
    auto *offsets = reinterpret_cast<std::uint32_t *>(ws);
    ws += align256(hist_n * 4u);
    void *scan_ws = ws;
    ws += scan_workspace_bytes(hist_n);
    std::uint32_t *tmp_keys = nullptr, *tmp_vals = nullptr;
    if (passes >= 2u) {
        tmp_keys = reinterpret_cast<std::uint32_t *>(ws);
        ws += align256(count * 4u);
        tmp_vals = reinterpret_cast<std::uint32_t *>(ws);
    }
    // the last pass lands in keys_out / vals_out
    const std::uint32_t *src_k = keys_in, *src_v = vals_in;
    for (std::uint32_t p = 0; p < passes; ++p) {
        const bool last = p + 1u == passes;
        const bool to_out = ((passes - 1u - p) % 2u) == 0u;
        std::uint32_t *dst_k = to_out ? keys_out : tmp_keys;
        std::uint32_t *dst_v = to_out ? vals_out : tmp_vals;
        (void)last;
        PassArgs a{src_k, src_v, dst_k, dst_v, hist, static_cast<std::uint32_t>(count), tiles, p * 8u};
        hipLaunchKernelGGL(radix_histogram, dim3(tiles), dim3(kSortThreads), 0, stream, a);
        int rc = exclusive_scan_u32(hist, offsets, hist_n, scan_ws, stream);
        if (rc != CX_STATUS_SUCCESS) return rc;
        a.hist = offsets;
        hipLaunchKernelGGL(radix_scatter, dim3(tiles), dim3(kSortThreads), 0, stream, a);
        rc = check_launch("radix_sort_pass");
        if (rc != CX_STATUS_SUCCESS) return rc;
        src_k = dst_k;
        src_v = dst_v;
    }
    return CX_STATUS_SUCCESS;
}

} // namespace cx

extern "C" int cx_sort_pairs_workspace(uint64_t count, uint32_t key_bits, uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (bytes == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_sort_pairs_workspace: null bytes");
    if (key_bits == 0u || key_bits > 32u) return fail(CX_STATUS_INVALID_SHAPE, "cx_sort_pairs_workspace: key_bits must be 1..32");
    *bytes = sort_pairs_workspace_bytes(count, key_bits);
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_sort_pairs(const uint32_t *keys_in, const uint32_t *vals_in, uint32_t *keys_out,
                             uint32_t *vals_out, uint64_t count, uint32_t key_bits, void *workspace,
                             uint64_t workspace_bytes, void *stream) {
    using namespace cx;
    clear_error();
    if (count != 0u && (keys_in == nullptr || keys_out == nullptr || vals_out == nullptr
                        || (workspace == nullptr && workspace_bytes != 0u)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_sort_pairs: null buffer");
    if (keys_out == keys_in || vals_out == vals_in || static_cast<void *>(keys_out) == vals_out)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_sort_pairs: outputs must not alias the inputs or each other");
    return sort_pairs(keys_in, vals_in, keys_out, vals_out, count, key_bits, workspace,
                      workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int cx_exclusive_scan_u32_workspace(uint64_t count, uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (bytes == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_exclusive_scan_u32_workspace: null bytes");
    *bytes = scan_workspace_bytes(count);
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_exclusive_scan_u32(const uint32_t *in, uint32_t *out, uint64_t count, void *workspace,
                                     uint64_t workspace_bytes, void *stream) {
    using namespace cx;
    clear_error();
    if (count != 0u && (in == nullptr || out == nullptr || workspace == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_exclusive_scan_u32: null buffer");
    if (workspace_bytes < scan_workspace_bytes(count))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_exclusive_scan_u32: workspace too small");
    return exclusive_scan_u32(in, out, count, workspace, static_cast<hipStream_t>(stream));
}
