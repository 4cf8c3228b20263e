// bell_spmm.hip -- Blocked-ELL SpMM on gfx950.
//
// MFMA path (bf16 values, bf16 weights, 32x32 blocks, N a multiple of 64):
//   * the weight panel is packed once per weight generation (cx_bell_pack_rhs) from
//     row-major K x N into fragment order: per 32-gene block column, 32-column tile and
//     K half, the 64 lanes' 16-byte B operands one after another, so a wave reads each
//     1 KB piece contiguously (the role of the reference's packed dense operand,
//     src/compute/math/packed_dense_operand.cu:131-260);
//   * values are row-major [rows][ell_cols] or block-major (CX_BELL_BLOCK_MAJOR_VALUES:
//     every 32x32 block's 2 KB contiguous); the kernels take the row and slot pitches;
//   * one workgroup owns one 32-row block; wave w owns output columns [64w, 64w+64)
//     as two 32x32 fp32 accumulator tiles;
//   * per valid ELL slot each lane loads its 16-byte A fragment (8 bf16 of one row of
//     the 32x32 value block) and 16-byte B fragments straight from the packed panel,
//     and issues v_mfma_f32_32x32x16_bf16 (two K steps of 16 per block); empty slots
//     (0xffffffff) are skipped without touching their values;
//   * row blocks are visited in an XCD-major order so consecutive row blocks of the
//     schedule share one XCD's L2 (the weight panel is re-read from L2, not HBM).
// Quantized path (codes of any width, 32x32 blocks, f32 W, N a multiple of 64): fp32 matrix
// cores, bell_spmm_quant_mfma below.
// Generic path (any other dtype / block size / N): one wave per row,
// lanes over output columns, slots in order, decoded with the codec exactly as
// quantized_blocked_ell_spmm_fwd_kernel_ does
// (src/compute/sparse/project/kernels/quantized_blocked_ell_spmm_fwd_kernel_.cuh:1-39).
#include "cx_common.hpp"

typedef __bf16 cx_bf16x8 __attribute__((ext_vector_type(8)));
typedef float cx_floatx16 __attribute__((ext_vector_type(16)));

namespace cx {
namespace {

constexpr std::uint32_t kInvalidBlock = 0xffffffffu;

struct BellArgs {
    const std::uint32_t *block_col_idx;
    const void *values;
    const std::uint8_t *packed;
    const float *scales;
    const float *offsets;
    const float *row_offsets;
    const void *rhs;
    std::int64_t rhs_ld;
    float *out;
    std::int64_t out_ld;
    std::uint32_t rows;
    std::uint32_t cols;
    std::uint32_t block_size;
    std::uint32_t ell_cols;
    std::uint32_t row_stride_bytes;
    // unquantized values: bytes between two rows of one row block's values, bytes between
    // two slots of one row, and the layout (row-major: ell_cols * size and block_size * size;
    // block-major: block_size * size and block_size^2 * size)
    std::uint32_t a_row_bytes;
    std::uint32_t a_slot_bytes;
    std::uint32_t block_major;
    // quantized matrix-core forms: row block of workgroup slot i (an XCD-major slot), or
    // none (the slot's own row block)
    const std::uint32_t *rb_order;
    Epilogue ep;
};

// Byte offset, within one block column's slice of the fragment-order panel
// (cx_bell_pack_rhs), of lane `lane`'s 16-byte B operand for 32-column tile `tile`, K half
// `half`.
__device__ __forceinline__ std::uint32_t panel_frag(std::uint32_t tile, std::uint32_t half, int lane) {
    return ((tile * 2u + half) * 64u + static_cast<std::uint32_t>(lane)) * 16u;
}

// Row block handled by workgroup `wg` of `count`: XCD-major so that the row blocks a
// single XCD processes are contiguous in the matrix (dispatch places wg on XCD wg % 8).
__device__ __forceinline__ std::uint32_t xcd_major(std::uint32_t wg, std::uint32_t count) {
    constexpr std::uint32_t kXcds = 8;
    const std::uint32_t per = count / kXcds;
    const std::uint32_t full = per * kXcds;
    if (wg >= full) return wg; // ragged tail keeps its natural index
    return (wg % kXcds) * per + wg / kXcds;
}

using rsrc_t = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, std::uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

// Bytes of row block rb's bf16 values (both layouts start it at rb * 32 * ell_cols
// elements): row-major, the rows the matrix has; block-major, whole blocks.
__device__ __forceinline__ std::uint32_t a_block_row_bytes(const BellArgs &a, std::uint32_t rb) {
    return a.block_major != 0u ? a.ell_cols * 64u : min(32u, a.rows - rb * 32u) * a.ell_cols * 2u;
}

// 16 bytes at voffset (per lane) + soffset (wave-uniform, kept in an SGPR so the per-step
// address needs no VALU arithmetic).
__device__ __forceinline__ cx_bf16x8 load_frag(rsrc_t r, std::uint32_t byte_offset,
                                               std::uint32_t uniform_offset = 0u) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(byte_offset),
                                                         static_cast<int>(uniform_offset), 0);
    cx_bf16x8 f;
    __builtin_memcpy(&f, &v, 16);
    return f;
}

// Operand fragments of one ELL slot for one wave: A (this lane's row, two K halves) and
// B (two 32-column tiles x two K halves).
struct SlotFrags {
    cx_bf16x8 a[2];
    cx_bf16x8 b[2][2];
};

template<int kN>
__global__ __launch_bounds__(kN) void bell_spmm_mfma(BellArgs a, const std::uint16_t *packed_rhs,
                                                     std::uint32_t panel_bytes,
                                                     const std::uint32_t *rb_list) {
    constexpr int kTilesPerWave = 2; // 64 output columns per wave
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const std::uint32_t row_blocks = (a.rows + 31u) / 32u;
    // a listed subset of row blocks (the planner's singletons), or all in XCD-major order
    const std::uint32_t rb = rb_list != nullptr ? rb_list[blockIdx.x] : xcd_major(blockIdx.x, gridDim.x);
    if (rb >= row_blocks) return;
    const std::uint32_t width = a.ell_cols / 32u;
    const std::uint32_t *slots = a.block_col_idx + static_cast<std::uint64_t>(rb) * width;

    const int m = lane % 32;         // A row / B,D column within the tile
    const int kq = (lane / 32) * 8;  // first K element of this lane's fragment
    const int n0 = wave * 64;
    // A: this row block's value rows (rows past the matrix read as 0 from the buffer)
    const rsrc_t ra = make_rsrc(static_cast<const std::uint16_t *>(a.values)
                                    + static_cast<std::uint64_t>(rb) * 32u * a.ell_cols,
                                a_block_row_bytes(a, rb));
    const rsrc_t rbp = make_rsrc(packed_rhs, panel_bytes);
    const std::uint32_t a_lane = static_cast<std::uint32_t>(m) * a.a_row_bytes + static_cast<std::uint32_t>(kq) * 2u;

    auto load_slot = [&](SlotFrags &f, std::uint32_t s, std::uint32_t bc) {
        const std::uint32_t ao = a_lane + s * a.a_slot_bytes;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) f.a[kc] = load_frag(ra, ao + static_cast<std::uint32_t>(kc) * 32u);
        const std::uint32_t bo = bc * static_cast<std::uint32_t>(kN) * 64u;
#pragma unroll
        for (int t = 0; t < kTilesPerWave; ++t)
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
                f.b[t][kc] = load_frag(rbp, bo + panel_frag(static_cast<std::uint32_t>(wave * kTilesPerWave + t),
                                                            static_cast<std::uint32_t>(kc), lane));
    };

    cx_floatx16 acc[kTilesPerWave];
#pragma unroll
    for (int t = 0; t < kTilesPerWave; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;

    auto mfma_slot = [&](const SlotFrags &f) {
#pragma unroll
        for (int t = 0; t < kTilesPerWave; ++t)
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[kc], f.b[t][kc], acc[t], 0, 0, 0);
    };

    // Valid slots of each 64-slot chunk are walked in order; the next valid slot's
    // fragments load (ping-pong registers) while the current slot's MFMAs run. Empty
    // slots (0xffffffff) are never read.
    for (std::uint32_t base = 0; base < width; base += kWave) {
        const std::uint32_t cnt = min(static_cast<std::uint32_t>(kWave), width - base);
        const std::uint32_t sid = static_cast<std::uint32_t>(lane) < cnt ? slots[base + lane] : kInvalidBlock;
        unsigned long long valid = __ballot(sid != kInvalidBlock);
        if (valid == 0ull) continue;
        SlotFrags f0, f1;
        std::uint32_t s = static_cast<std::uint32_t>(__builtin_ctzll(valid));
        load_slot(f0, base + s, static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(sid), static_cast<int>(s))));
        valid &= valid - 1ull;
        // The prefetch is issued unconditionally (the last one re-reads the current slot):
        // with no branch around it, each wait covers only the slot about to be used.
        for (;;) {
            const bool more0 = valid != 0ull;
            if (more0) s = static_cast<std::uint32_t>(__builtin_ctzll(valid));
            load_slot(f1, base + s, static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(sid), static_cast<int>(s))));
            valid &= valid - 1ull;
            __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of these MFMAs
            mfma_slot(f0);
            __builtin_amdgcn_sched_barrier(0);
            if (!more0) break;
            const bool more1 = valid != 0ull;
            if (more1) s = static_cast<std::uint32_t>(__builtin_ctzll(valid));
            load_slot(f0, base + s, static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(sid), static_cast<int>(s))));
            valid &= valid - 1ull;
            __builtin_amdgcn_sched_barrier(0);
            mfma_slot(f1);
            __builtin_amdgcn_sched_barrier(0);
            if (!more1) break;
        }
    }

    // D layout: lane holds column (lane % 32); element i is row 8*(i/4) + 4*(lane/32) + i%4.
#pragma unroll
    for (int t = 0; t < kTilesPerWave; ++t) {
        const int col = n0 + t * 32 + m;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const std::uint32_t r = rb * 32u + 8u * (i / 4) + 4u * (lane / 32) + (i % 4);
            if (r < a.rows)
                a.out[static_cast<std::int64_t>(r) * a.out_ld + col] =
                    a.ep.active ? epilogue_value(a.ep, acc[t][i], r, col) : acc[t][i];
        }
    }
}


// Grouped MFMA path. One workgroup per planner group of 2..4 row blocks whose valid
// block-column lists are prefixes of the longest member's (cx_bell_plan_groups). Wave w owns
// member w across all N output columns (N/32 accumulator tiles). At step k every member
// uses the group's k-th block column, so its N x 32 panel slice is loaded from the packed
// panel once per group into an LDS ring of three slices (column stride 80 B: 8 consecutive
// lanes' 16-byte reads hit distinct banks). Panel slices are issued three steps before use
// (three register sets, then LDS), the members' A fragments (their k-th valid slot) two.
constexpr int kGroupWaves = 4;
constexpr int kPanelColStride = 80;
constexpr int kRing = 3;

using lds_void = __attribute__((address_space(3))) void *;

template<int kN>
__global__ __launch_bounds__(kWave *kGroupWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void bell_spmm_mfma_grouped(BellArgs a, const std::uint16_t *packed_rhs, std::uint32_t panel_bytes,
                            const std::uint32_t *order, const std::uint32_t *group_offsets,
                            std::uint32_t group_count, std::uint32_t grouped_row_blocks) {
    constexpr int kTiles = kN / 32;
    constexpr int kSlice = kN * kPanelColStride;
    constexpr int kChunks = kN * 4;  // 16-byte chunks of one N x 32 bf16 slice
    constexpr int kThreads = kWave * kGroupWaves;
    constexpr int kLoadIters = (kChunks + kThreads - 1) / kThreads;
    __shared__ __attribute__((aligned(16))) unsigned char bslice[kRing][kSlice];
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t wave = static_cast<std::uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave)));
    // XCD-major: each XCD takes a contiguous range of the planner's order, whose neighbouring
    // groups share block columns, so the panel slices in use stay in that XCD's L2.
    // Workgroups past the groups take the single row blocks, one each.
    const std::uint32_t wg = xcd_major(blockIdx.x, gridDim.x);
    const bool single = wg >= group_count;
    const std::uint32_t g0 = single ? grouped_row_blocks + (wg - group_count) : group_offsets[wg];
    const std::uint32_t g1 = single ? g0 + 1u : group_offsets[wg + 1];
    const std::uint32_t members = g1 - g0;
    const std::uint32_t leader = order[g1 - 1u];
    const bool active = wave < members;
    const std::uint32_t rb = active ? order[g0 + wave] : leader;
    const std::uint32_t width = a.ell_cols / 32u;
    const std::uint32_t lead_sid = static_cast<std::uint32_t>(lane) < width
        ? a.block_col_idx[static_cast<std::uint64_t>(leader) * width + lane] : kInvalidBlock;
    const std::uint32_t own_sid = static_cast<std::uint32_t>(lane) < width
        ? a.block_col_idx[static_cast<std::uint64_t>(rb) * width + lane] : kInvalidBlock;
    unsigned long long lead_valid = __ballot(lead_sid != kInvalidBlock);
    unsigned long long own_valid = active ? __ballot(own_sid != kInvalidBlock) : 0ull;
    const std::uint32_t steps = static_cast<std::uint32_t>(__popcll(lead_valid));
    const std::uint32_t own_steps = static_cast<std::uint32_t>(__popcll(own_valid));

    const int m = lane % 32;
    const int kq = (lane / 32) * 8;
    const rsrc_t ra = make_rsrc(static_cast<const std::uint16_t *>(a.values)
                                    + static_cast<std::uint64_t>(rb) * 32u * a.ell_cols,
                                a_block_row_bytes(a, rb));
    const rsrc_t rbp = make_rsrc(packed_rhs, panel_bytes);
    const std::uint32_t a_lane = static_cast<std::uint32_t>(m) * a.a_row_bytes + static_cast<std::uint32_t>(kq) * 2u;

    cx_floatx16 acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;

    // the group's next block column (after the last one: repeats it; never stored)
    std::uint32_t last_bc = 0u;
    auto next_lead = [&]() {
        if (lead_valid != 0ull) {
            const std::uint32_t s = static_cast<std::uint32_t>(__builtin_ctzll(lead_valid));
            lead_valid &= lead_valid - 1ull;
            last_bc = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lead_sid), static_cast<int>(s)));
        }
        return last_bc;
    };
    auto next_own = [&]() {
        const std::uint32_t s = own_valid != 0ull ? static_cast<std::uint32_t>(__builtin_ctzll(own_valid)) : 0u;
        own_valid &= own_valid - 1ull;
        return s;
    };
    struct BRegs { uint4 c[kLoadIters]; };
    auto load_b = [&](BRegs &b, std::uint32_t bc) {
#pragma unroll
        for (int i = 0; i < kLoadIters; ++i) {
            const std::uint32_t c = threadIdx.x + static_cast<std::uint32_t>(i) * kThreads;
            const std::uint32_t cc = c < static_cast<std::uint32_t>(kChunks) ? c : 0u;
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(
                rbp, static_cast<int>(cc * 16u), static_cast<int>(bc * static_cast<std::uint32_t>(kN) * 64u), 0);
            __builtin_memcpy(&b.c[i], &v, 16);
        }
    };
    // chunk c of the slice is fragment (tile c / 128, K half (c / 64) % 2) of lane c % 64:
    // column 32 tile + (c % 32), genes 16 half + 8 ((c % 64) / 32) .. + 7
    auto store_b = [&](const BRegs &b, std::uint32_t slot) {
#pragma unroll
        for (int i = 0; i < kLoadIters; ++i) {
            const std::uint32_t c = threadIdx.x + static_cast<std::uint32_t>(i) * kThreads;
            const std::uint32_t col = (c / 128u) * 32u + c % 32u;
            const std::uint32_t kchunk = ((c / 64u) % 2u) * 2u + (c % 64u) / 32u;
            if (c < static_cast<std::uint32_t>(kChunks))
                *reinterpret_cast<uint4 *>(&bslice[slot][col * kPanelColStride + kchunk * 16u]) = b.c[i];
        }
    };
    auto load_a = [&](cx_bf16x8 (&af)[2], std::uint32_t s) {
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
            af[kc] = load_frag(ra, a_lane + static_cast<std::uint32_t>(kc) * 32u, s * a.a_slot_bytes);
    };
    auto mfma_step = [&](const cx_bf16x8 (&af)[2], std::uint32_t slot) {
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                cx_bf16x8 bf;
                __builtin_memcpy(&bf, &bslice[slot][(t * 32 + m) * kPanelColStride + (kq + kc * 16) * 2], 16);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kc], bf, acc[t], 0, 0, 0);
            }
    };

    if (steps != 0u) {
        // Slices and A fragments both run two steps ahead: slice j lives in register set
        // j % 3 from its issue (step j - 3) until it is stored to LDS slot j % 3 (end of step
        // j - 1); A(j) lives in a[j % 3] from step j - 2. Both stream from L2/HBM, and a step
        // (16 MFMAs per wave at N = 256) is far shorter than their latency.
        BRegs b0, b1, b2;
        cx_bf16x8 a0[2], a1[2], a2[2];
        load_b(b0, next_lead());   // slice 0
        load_b(b1, next_lead());   // slice 1
        load_b(b2, next_lead());   // slice 2
        load_a(a0, next_own());
        load_a(a1, next_own());
        store_b(b0, 0u);
        __syncthreads();
        std::uint32_t k = 0, slot = 0;
        auto step = [&](BRegs &free_regs, BRegs &to_store, cx_bf16x8 (&a_cur)[2], cx_bf16x8 (&a_new)[2]) {
            load_b(free_regs, next_lead());     // slice k+3 (its set held slice k, stored last step)
            load_a(a_new, next_own());          // A(k+2)
            if (active && k < own_steps) mfma_step(a_cur, slot);
            const std::uint32_t nslot = slot + 1u == static_cast<std::uint32_t>(kRing) ? 0u : slot + 1u;
            if (k + 1u < steps) store_b(to_store, nslot);  // slice k+1
            __syncthreads();
            slot = nslot;
            ++k;
        };
        for (;;) {
            step(b0, b1, a0, a2);
            if (k >= steps) break;
            step(b1, b2, a1, a0);
            if (k >= steps) break;
            step(b2, b0, a2, a1);
            if (k >= steps) break;
        }
    }

    if (!active) return;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const int col = t * 32 + m;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const std::uint32_t r = rb * 32u + 8u * (i / 4) + 4u * (lane / 32) + (i % 4);
            if (r < a.rows)
                a.out[static_cast<std::int64_t>(r) * a.out_ld + col] =
                    a.ep.active ? epilogue_value(a.ep, acc[t][i], r, col) : acc[t][i];
        }
    }
}

// Grouped MFMA path by column slab (N = 128 with 4 waves, N = 256 with 8). Same groups, steps
// and sums as above, but wave w computes output columns [32w, 32w + 32) of every member. The
// members' A blocks (2 KB each per step) are shared through an LDS ring, loaded straight into
// LDS (buffer loads with the lds flag), and each wave's B fragments (its slab of the step's
// panel slice) come from the packed panel into registers; both run three steps ahead. Per
// group and step the LDS carries 8 KB of A, written once and read by every wave with
// conflict-free 16-byte reads, instead of a 16 KB slice read four times. A member without a
// step k skips its products. Per output element the products are accumulated in the same
// slot order as the other MFMA kernels, so the results are bitwise equal.

// s_waitcnt operand: vector memory count n (6 bits, split over two fields), lgkmcnt(0),
// expcnt unchecked
constexpr unsigned vmcnt_wait(int n) {
    return 0x0070u | (static_cast<unsigned>(n) & 15u) | ((static_cast<unsigned>(n) >> 4) << 14);
}

// 16 bytes per lane from a buffer straight into LDS at dst + lane * 16 (dst wave-uniform)
__device__ __forceinline__ void load_lds16(rsrc_t r, uint4 *dst, std::uint32_t voffset, std::uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void)dst, 16, voffset, soffset, 0, 0);
}

template<int kN, bool kBlockMajor, int kWaves>
__global__ __launch_bounds__(kWave *kWaves) __attribute__((amdgpu_waves_per_eu(kWaves / 2, kWaves / 2)))
void bell_spmm_mfma_slab(BellArgs a, const std::uint16_t *packed_rhs, std::uint32_t panel_bytes,
                         const std::uint32_t *order, const std::uint32_t *group_offsets,
                         std::uint32_t group_count, std::uint32_t grouped_row_blocks) {
    constexpr int kSlabTiles = kN / (32 * kWaves);
    static_assert(kSlabTiles >= 1, "a slab is at least one 32-column tile");
    constexpr int kPieces = 2 * kGroupWaves / kWaves;  // A pieces (member, half) per wave per step
    static_assert(kPieces == 1 || kPieces == 2, "4 or 8 waves");
    constexpr int kStepLoads = 2 * kSlabTiles + kPieces;  // vector loads one step issues: B, then A
    // Loads run three steps ahead; at the end of step k only the loads of steps k + 2 and k + 3
    // may still be in flight.
    constexpr unsigned kStepWait = vmcnt_wait(2 * kStepLoads);
    // The A ring: four separately declared slots ([member][K half][lane]), addressed with
    // compile-time slot numbers, so that the compiler can tell a read of one slot from the
    // LDS loads in flight into the others and adds no wait for those.
    __shared__ uint4 a_lds0[kGroupWaves][2][kWave];
    __shared__ uint4 a_lds1[kGroupWaves][2][kWave];
    __shared__ uint4 a_lds2[kGroupWaves][2][kWave];
    __shared__ uint4 a_lds3[kGroupWaves][2][kWave];
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t wave = static_cast<std::uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave)));
    const std::uint32_t wg = xcd_major(blockIdx.x, gridDim.x);
    const bool single = wg >= group_count;
    const std::uint32_t g0 = single ? grouped_row_blocks + (wg - group_count) : group_offsets[wg];
    const std::uint32_t g1 = single ? g0 + 1u : group_offsets[wg + 1];
    const std::uint32_t members = g1 - g0;
    const std::uint32_t leader = order[g1 - 1u];
    const std::uint32_t width = a.ell_cols / 32u;

    // slot lists: the leader's (the B sequence) and the two members whose A this wave loads
    // (member wave / 2 and 2 + wave / 2, K half wave % 2)
    const std::uint32_t lead_sid = static_cast<std::uint32_t>(lane) < width
        ? a.block_col_idx[static_cast<std::uint64_t>(leader) * width + lane] : kInvalidBlock;
    unsigned long long lead_valid = __ballot(lead_sid != kInvalidBlock);
    const std::uint32_t steps = static_cast<std::uint32_t>(__popcll(lead_valid));
    std::uint32_t own_steps[kGroupWaves];
    std::uint32_t rbs[kGroupWaves];
#pragma unroll
    for (int mm = 0; mm < kGroupWaves; ++mm) {
        const std::uint32_t rb = static_cast<std::uint32_t>(mm) < members ? order[g0 + mm] : leader;
        rbs[mm] = rb;
        const std::uint32_t sid = static_cast<std::uint32_t>(lane) < width
            ? a.block_col_idx[static_cast<std::uint64_t>(rb) * width + lane] : kInvalidBlock;
        own_steps[mm] = static_cast<std::uint32_t>(mm) < members ? static_cast<std::uint32_t>(__popcll(__ballot(sid != kInvalidBlock))) : 0u;
    }
    // this wave's A loads: pieces wave and wave + kWaves of the 8 (member, half) pieces, i.e.
    // members la and lb (4 waves) or la alone (8 waves), half kh (all wave-uniform)
    const std::uint32_t la = wave / 2u, lb = (wave + static_cast<std::uint32_t>(kWaves)) / 2u, kh = wave % 2u;
    struct ALoads {
        rsrc_t r;
        unsigned long long valid;
        std::uint32_t steps;
    };
    auto a_loads = [&](std::uint32_t mm) {
        const std::uint32_t rb = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(
            static_cast<int>(mm < members ? order[g0 + mm] : leader)));
        const std::uint32_t sid = static_cast<std::uint32_t>(lane) < width
            ? a.block_col_idx[static_cast<std::uint64_t>(rb) * width + lane] : kInvalidBlock;
        ALoads l;
        l.valid = mm < members ? __ballot(sid != kInvalidBlock) : 0ull;
        l.steps = static_cast<std::uint32_t>(__popcll(l.valid));
        l.r = make_rsrc(static_cast<const std::uint16_t *>(a.values) + static_cast<std::uint64_t>(rb) * 32u * a.ell_cols,
                        a_block_row_bytes(a, rb));
        return l;
    };
    ALoads ld_a = a_loads(la), ld_b;
    if constexpr (kPieces == 2) ld_b = a_loads(lb);
    const rsrc_t rbp = make_rsrc(packed_rhs, panel_bytes);
    const int m = lane % 32;
    const int kq = (lane / 32) * 8;
    // Row-major values: wave w loads K half kh (16 columns) of all 32 rows, lane by lane in
    // fragment order. Block-major values: wave w loads rows [16 kh, 16 kh + 16) whole, a
    // contiguous 1 KB, and lane l puts row 16 kh + l / 4's 16-byte chunk
    // (l % 4) ^ ((row / 4) % 4) at position l: each row's four chunks rotate by its quad, so
    // the fragment reads below (16 rows, one chunk) meet every bank once.
    std::uint32_t a_lane, a_read[2] = {0u, 0u};
    if constexpr (kBlockMajor) {
        const std::uint32_t r = kh * 16u + static_cast<std::uint32_t>(lane) / 4u;
        a_lane = r * 64u + ((static_cast<std::uint32_t>(lane) % 4u) ^ ((r / 4u) % 4u)) * 16u;
        const std::uint32_t mm_ = static_cast<std::uint32_t>(m), h = static_cast<std::uint32_t>(lane) / 32u;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
            a_read[kc] = mm_ * 4u + ((static_cast<std::uint32_t>(kc) * 2u + h) ^ ((mm_ / 4u) % 4u));
    } else {
        a_lane = (static_cast<std::uint32_t>(m) * a.ell_cols + static_cast<std::uint32_t>(kq) + kh * 16u) * 2u;
    }
    constexpr std::uint32_t kSlotBytes = kBlockMajor ? 2048u : 64u;

    cx_floatx16 acc[kGroupWaves][kSlabTiles];
#pragma unroll
    for (int mm = 0; mm < kGroupWaves; ++mm)
#pragma unroll
        for (int t = 0; t < kSlabTiles; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mm][t][i] = 0.0f;

    std::uint32_t last_bc = 0u;
    auto next_lead = [&]() {
        if (lead_valid != 0ull) {
            const std::uint32_t sl = static_cast<std::uint32_t>(__builtin_ctzll(lead_valid));
            lead_valid &= lead_valid - 1ull;
            last_bc = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lead_sid), static_cast<int>(sl)));
        }
        return last_bc;
    };
    struct BFrags { cx_bf16x8 f[kSlabTiles][2]; };
    auto load_b = [&](BFrags &b, std::uint32_t bc) {
#pragma unroll
        for (int t = 0; t < kSlabTiles; ++t)
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
                b.f[t][kc] = load_frag(rbp, panel_frag(wave * kSlabTiles + static_cast<std::uint32_t>(t),
                                                       static_cast<std::uint32_t>(kc), lane),
                                       bc * static_cast<std::uint32_t>(kN) * 64u);
    };
    using Slot = uint4[kGroupWaves][2][kWave];
    // A of the next step for members la, lb (K half kh) into a ring slot. Both loads are
    // always issued (a member without that step reloads its first slot into a part of the
    // ring nobody reads), so every step has the same count of loads in flight and the waits
    // below are exact.
    auto issue_one = [&](ALoads &l, std::uint32_t mm, Slot &slot) {
        const std::uint32_t sl = l.valid != 0ull ? static_cast<std::uint32_t>(__builtin_ctzll(l.valid)) : 0u;
        l.valid &= l.valid - 1ull;
        load_lds16(l.r, &slot[mm][kh][0], a_lane, sl * kSlotBytes);
    };
    auto issue_a = [&](Slot &slot) {
        issue_one(ld_a, la, slot);
        if constexpr (kPieces == 2) issue_one(ld_b, lb, slot);
    };
    // Barrier without a memory fence (a fence would wait for every LDS load in flight): the
    // waits before it are explicit, and the asm's memory clobber keeps LDS accesses on their
    // side of it.
    auto barrier = []() { asm volatile("s_barrier" ::: "memory"); };

    if (steps != 0u) {
        BFrags b0, b1, b2, b3;
        load_b(b0, next_lead());
        issue_a(a_lds0);
        load_b(b1, next_lead());
        issue_a(a_lds1);
        load_b(b2, next_lead());
        issue_a(a_lds2);
        __builtin_amdgcn_s_waitcnt(kStepWait);  // step 0's loads are in
        barrier();
        std::uint32_t k = 0;
        // step k reads set and slot k % 4 and loads B(k + 3), A(k + 3) into set and slot
        // (k + 3) % 4, the ones step k - 1 read (every wave has passed the barrier after it)
        auto step = [&](BFrags &b_cur, BFrags &b_new, Slot &slot, Slot &fill_slot) {
            __builtin_amdgcn_sched_barrier(0);
            load_b(b_new, next_lead());  // B(k + 3)
            __builtin_amdgcn_sched_barrier(0);
            issue_a(fill_slot);  // A(k + 3)
            __builtin_amdgcn_sched_barrier(0);
            // 4 waves: all members' A fragments first (one LDS round trip), then their
            // products; 8 waves (128 registers): each member's fragments just before its own
            auto read_a = [&](cx_bf16x8 (&f)[2], int mm) {
#pragma unroll
                for (int kc = 0; kc < 2; ++kc) {
                    if constexpr (kBlockMajor)
                        f[kc] = __builtin_bit_cast(cx_bf16x8, (&slot[mm][0][0])[a_read[kc]]);
                    else
                        f[kc] = __builtin_bit_cast(cx_bf16x8, slot[mm][kc][lane]);
                }
            };
            constexpr bool kHoist = kWaves == 4;
            cx_bf16x8 af[kHoist ? kGroupWaves : 1][2];
            if constexpr (kHoist) {
#pragma unroll
                for (int mm = 0; mm < kGroupWaves; ++mm) read_a(af[mm], mm);
            }
#pragma unroll
            for (int mm = 0; mm < kGroupWaves; ++mm) {
                if (k < own_steps[mm]) {
                    if constexpr (!kHoist) read_a(af[0], mm);
#pragma unroll
                    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
                        for (int t = 0; t < kSlabTiles; ++t)
                            acc[mm][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kHoist ? mm : 0][kc], b_cur.f[t][kc],
                                                                                 acc[mm][t], 0, 0, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            // B(k + 1) and A(k + 1) (issued at step k - 2) must be in for the next step, and this
            // step's LDS reads done before the slot is refilled
            __builtin_amdgcn_s_waitcnt(kStepWait);
            barrier();
            ++k;
        };
        for (;;) {
            step(b0, b3, a_lds0, a_lds3);
            if (k >= steps) break;
            step(b1, b0, a_lds1, a_lds0);
            if (k >= steps) break;
            step(b2, b1, a_lds2, a_lds1);
            if (k >= steps) break;
            step(b3, b2, a_lds3, a_lds2);
            if (k >= steps) break;
        }
        // the last steps' A loads are still landing in LDS: nothing may leave before them
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
    }

    // one call per member (a loop over members with the accumulators indexed by it is not
    // unrolled at this size, which would put them in scratch)
    auto store_member = [&](const cx_floatx16 (&acc_m)[kSlabTiles], std::uint32_t rb) {
#pragma unroll
        for (int t = 0; t < kSlabTiles; ++t) {
            const int col = (static_cast<int>(wave) * kSlabTiles + t) * 32 + m;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const std::uint32_t r = rb * 32u + 8u * (i / 4) + 4u * (lane / 32) + (i % 4);
                if (r < a.rows)
                    a.out[static_cast<std::int64_t>(r) * a.out_ld + col] =
                        a.ep.active ? epilogue_value(a.ep, acc_m[t][i], r, col) : acc_m[t][i];
            }
        }
    };
    store_member(acc[0], rbs[0]);
    if (members > 1u) store_member(acc[1], rbs[1]);
    if (members > 2u) store_member(acc[2], rbs[2]);
    if (members > 3u) store_member(acc[3], rbs[3]);
}

// Column-contiguous panel [ceil(k/32)][n][32] (the dense head of the quantized CSR path
// reads this form): one thread per packed element (kb, col, kk).
__global__ void pack_rhs_kernel(const std::uint16_t *rhs, std::int64_t rhs_ld, std::uint32_t k,
                                std::uint32_t n, std::uint16_t *packed) {
    const std::uint64_t idx = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x;
    const std::uint32_t kblocks = (k + 31u) / 32u;
    const std::uint64_t total = static_cast<std::uint64_t>(kblocks) * n * 32u;
    if (idx >= total) return;
    const std::uint32_t kk = static_cast<std::uint32_t>(idx % 32u);
    const std::uint32_t col = static_cast<std::uint32_t>((idx / 32u) % n);
    const std::uint32_t kb = static_cast<std::uint32_t>(idx / (32ull * n));
    const std::uint32_t gene = kb * 32u + kk;
    packed[idx] = gene < k ? rhs[static_cast<std::int64_t>(gene) * rhs_ld + col] : 0;
}

// Fragment-order panel (cx_bell_pack_rhs): element idx of block column kb is
// ((tile * 2 + half) * 64 + lane) * 8 + i, holding column 32 tile + lane % 32 and gene
// 32 kb + 16 half + 8 (lane / 32) + i. One thread per element.
__global__ void pack_rhs_frag_kernel(const std::uint16_t *rhs, std::int64_t rhs_ld, std::uint32_t k,
                                     std::uint32_t n, std::uint16_t *packed) {
    const std::uint64_t idx = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x;
    const std::uint32_t kblocks = (k + 31u) / 32u;
    const std::uint64_t total = static_cast<std::uint64_t>(kblocks) * n * 32u;
    if (idx >= total) return;
    const std::uint32_t kb = static_cast<std::uint32_t>(idx / (32ull * n));
    const std::uint32_t e = static_cast<std::uint32_t>(idx % (32ull * n));
    const std::uint32_t i = e % 8u, lane = (e / 8u) % 64u, half = (e / 512u) % 2u, tile = e / 1024u;
    const std::uint32_t col = tile * 32u + lane % 32u;
    const std::uint32_t gene = kb * 32u + half * 16u + (lane / 32u) * 8u + i;
    packed[idx] = gene < k ? rhs[static_cast<std::int64_t>(gene) * rhs_ld + col] : 0;
}

// Row-major -> block-major values (CX_BELL_BLOCK_MAJOR_VALUES), one thread per element of
// the output; rows past the matrix are zero.
template<typename T>
__global__ void block_major_kernel(const T *values, std::uint32_t rows, std::uint32_t bs,
                                   std::uint32_t ell_cols, std::uint64_t total, T *out) {
    const std::uint64_t idx = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x;
    if (idx >= total) return;
    const std::uint64_t block = idx / (static_cast<std::uint64_t>(bs) * bs);  // rb * width + slot
    const std::uint32_t within = static_cast<std::uint32_t>(idx % (static_cast<std::uint64_t>(bs) * bs));
    const std::uint32_t width = ell_cols / bs;
    const std::uint64_t rb = block / width;
    const std::uint32_t slot = static_cast<std::uint32_t>(block % width);
    const std::uint64_t row = rb * bs + within / bs;
    out[idx] = row < rows ? values[row * ell_cols + static_cast<std::uint64_t>(slot) * bs + within % bs] : T{};
}

template<typename T>
__device__ __forceinline__ float load_as_float(const void *p, std::uint64_t i, std::uint32_t dtype) {
    if (dtype == CELLERATOR_DTYPE_F32) return static_cast<const float *>(p)[i];
    const std::uint16_t bits = static_cast<const std::uint16_t *>(p)[i];
    return dtype == CELLERATOR_DTYPE_BF16 ? bf2f(bits) : h2f(bits);
}

// Reference-semantics kernel: row per wave, lanes over output columns, slots in order.
__global__ __launch_bounds__(256) void bell_spmm_generic(BellArgs a, std::uint32_t value_dtype,
                                                         std::uint32_t rhs_dtype, std::uint32_t bits,
                                                         std::uint32_t policy, std::int64_t n) {
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t row = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (row >= a.rows) return;
    const std::uint32_t bs = a.block_size;
    const std::uint32_t width = a.ell_cols / bs;
    const std::uint32_t rb = row / bs;
    const float row_offset = (bits != 0u && policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET
                              && a.row_offsets != nullptr) ? a.row_offsets[row] : 0.0f;
    for (std::int64_t c0 = 0; c0 < n; c0 += kWave) {
        const std::int64_t c = c0 + lane;
        float acc = 0.0f;
        for (std::uint32_t s = 0; s < width; ++s) {
            const std::uint32_t bc = a.block_col_idx[static_cast<std::uint64_t>(rb) * width + s];
            if (bc == kInvalidBlock) continue;
            for (std::uint32_t kk = 0; kk < bs; ++kk) {
                const std::uint64_t col = static_cast<std::uint64_t>(bc) * bs + kk;
                if (col >= a.cols) break;
                const std::uint32_t slot = s * bs + kk;
                float x;
                if (bits != 0u) {
                    const std::uint32_t cpb = 8u / bits;
                    const std::uint8_t byte = a.packed[static_cast<std::uint64_t>(row) * a.row_stride_bytes
                                                       + slot / cpb];
                    const std::uint32_t code = (byte >> ((slot % cpb) * bits)) & ((1u << bits) - 1u);
                    const float scale = a.scales != nullptr ? a.scales[col] : 1.0f;
                    const float offset = policy == CX_DECODE_PER_GENE_AFFINE
                        ? (a.offsets != nullptr ? a.offsets[col] : 0.0f)
                        : row_offset;
                    x = __builtin_fmaf(static_cast<float>(code), scale, offset);
                } else {
                    const std::uint64_t vi = a.block_major != 0u
                        ? ((static_cast<std::uint64_t>(rb) * width + s) * bs + row % bs) * bs + kk
                        : static_cast<std::uint64_t>(row) * a.ell_cols + slot;
                    x = load_as_float<float>(a.values, vi, value_dtype);
                }
                if (c < n) {
                    const float w = load_as_float<float>(a.rhs, col * a.rhs_ld + c, rhs_dtype);
                    acc = __builtin_fmaf(x, w, acc);
                }
            }
        }
        if (c < n)
            a.out[static_cast<std::int64_t>(row) * a.out_ld + c] =
                a.ep.active ? epilogue_value(a.ep, acc, row, c) : acc;
    }
}

// Quantized Blocked-ELL on the matrix cores (codes of 1/2/4/8 bits, either decode policy,
// 32x32 blocks, f32 W, N a multiple of 64): the reference's quantized projection
// (quantized_blocked_ell_spmm_fwd_f32, src/compute/sparse/project/project.cu:108-168) with
// every value decoded exactly as its kernel does, fma(code, scale, offset) in fp32, and the
// products on v_mfma_f32_32x32x2_f32 (fp32 operands, fp32 accumulation: only the summation
// order differs). One workgroup of 4 waves per 32-row block; wave w takes the 64-column
// chunks w, w + 4, ... as two 32x32 accumulator tiles. Per valid slot (block column bc),
// lane l (row m = l % 32 of the block, K parity h = l / 32) loads its row's 32 codes of the
// block (kBits dwords) and the (scale, offset) of gene bc * 32 + m, and per K step kk of 2
// (genes 2kk, 2kk + 1) decodes the code of gene 2kk + h with that gene's metadata taken from
// lanes 2kk and 2kk + 1 (readlane), so A[m][h] = x, and loads B[h][n] = W[gene][column n].
// Genes past `cols` (a last partial block column) read as 0 in both operands. The next valid
// slot's codes, metadata and W are loaded while the current slot's matrix instructions run.
template<int kBits>
struct QuantSlot {
    std::uint32_t codes[kBits];  // this lane's row: the block's 32 codes, kBits * 32 bits
    float meta[2];               // scale and offset of gene bc * 32 + lane % 32
    float w[16][2];              // B operands: K step x 32-column tile
};

template<int kBits, int kPolicy>
__global__ __launch_bounds__(256) void bell_spmm_quant_mfma(BellArgs a, std::int64_t n) {
    constexpr int kTiles = 2;  // 64 output columns per wave and chunk
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const std::uint32_t row_blocks = (a.rows + 31u) / 32u;
    const std::uint32_t slot = xcd_major(blockIdx.x, gridDim.x);
    const std::uint32_t rb = a.rb_order != nullptr ? a.rb_order[slot] : slot;
    if (rb >= row_blocks) return;
    const std::uint32_t width = a.ell_cols / 32u;
    const std::uint32_t *slots = a.block_col_idx + static_cast<std::uint64_t>(rb) * width;
    const int m = lane % 32;
    const int h = lane / 32;
    const std::uint32_t row = rb * 32u + static_cast<std::uint32_t>(m);
    // this row block's codes; rows past the matrix read as 0 (their sums are not stored)
    const std::uint32_t block_rows = min(32u, a.rows - rb * 32u);
    const rsrc_t rc = make_rsrc(a.packed + static_cast<std::uint64_t>(rb) * 32u * a.row_stride_bytes,
                                block_rows * a.row_stride_bytes);
    const std::uint32_t code_lane = static_cast<std::uint32_t>(m) * a.row_stride_bytes;
    const float row_offset = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET && row < a.rows ? a.row_offsets[row] : 0.0f;
    const float *w = static_cast<const float *>(a.rhs);

    for (std::int64_t n0 = static_cast<std::int64_t>(wave) * 64; n0 < n; n0 += 256) {
        auto load_slot = [&](QuantSlot<kBits> &f, std::uint32_t s, std::uint32_t bc) {
            const std::uint32_t co = code_lane + s * static_cast<std::uint32_t>(kBits) * 4u;
            if constexpr (kBits >= 4) {
#pragma unroll
                for (int q = 0; q < kBits / 4; ++q) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rc, static_cast<int>(co) + 16 * q, 0, 0);
                    f.codes[4 * q] = v[0]; f.codes[4 * q + 1] = v[1]; f.codes[4 * q + 2] = v[2]; f.codes[4 * q + 3] = v[3];
                }
            } else {
#pragma unroll
                for (int q = 0; q < kBits; ++q)
                    f.codes[q] = static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rc, static_cast<int>(co) + 4 * q, 0, 0));
            }
            const std::uint32_t g = bc * 32u + static_cast<std::uint32_t>(m);
            const bool in = g < a.cols;
            f.meta[0] = in && a.scales != nullptr ? a.scales[g] : (in ? 1.0f : 0.0f);
            f.meta[1] = kPolicy == CX_DECODE_PER_GENE_AFFINE && in && a.offsets != nullptr ? a.offsets[g] : 0.0f;
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                const std::uint32_t gk = bc * 32u + static_cast<std::uint32_t>(2 * kk + h);
#pragma unroll
                for (int t = 0; t < kTiles; ++t)
                    f.w[kk][t] = gk < a.cols ? w[static_cast<std::int64_t>(gk) * a.rhs_ld + n0 + 32 * t + m] : 0.0f;
            }
        };

        cx_floatx16 acc[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;

        auto mfma_slot = [&](const QuantSlot<kBits> &f, std::uint32_t bc) {
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                // gene 2kk + h of the block: its code in this lane's row, its metadata from
                // lane 2kk + h (the lane that loaded gene 2kk + h's pair)
                const int bit = (2 * kk) * kBits;  // first bit of gene 2kk; gene 2kk + 1 follows
                const std::uint32_t word = f.codes[bit / 32];
                const std::uint32_t code = (word >> ((bit % 32) + h * kBits)) & ((1u << kBits) - 1u);
                const float se = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f.meta[0]), 2 * kk));
                const float so = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f.meta[0]), 2 * kk + 1));
                const float oe = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f.meta[1]), 2 * kk));
                const float oo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f.meta[1]), 2 * kk + 1));
                const float scale = h != 0 ? so : se;
                const float offset = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET ? row_offset : (h != 0 ? oo : oe);
                const bool in = bc * 32u + static_cast<std::uint32_t>(2 * kk + h) < a.cols;
                const float x = in ? __builtin_fmaf(static_cast<float>(code), scale, offset) : 0.0f;
#pragma unroll
                for (int t = 0; t < kTiles; ++t)
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, f.w[kk][t], acc[t], 0, 0, 0);
            }
        };

        // valid slots in order; the next one's operands load while the current one's run
        std::uint32_t s = 0u;
        while (s < width && slots[s] == kInvalidBlock) ++s;
        if (s < width) {
            QuantSlot<kBits> f0, f1;
            std::uint32_t bc0 = slots[s];
            load_slot(f0, s, bc0);
            for (;;) {
                std::uint32_t t1 = s + 1u;
                while (t1 < width && slots[t1] == kInvalidBlock) ++t1;
                const bool more = t1 < width;
                const std::uint32_t bc1 = more ? slots[t1] : bc0;
                load_slot(f1, more ? t1 : s, bc1);
                __builtin_amdgcn_sched_barrier(0);
                mfma_slot(f0, bc0);
                __builtin_amdgcn_sched_barrier(0);
                if (!more) break;
                s = t1;
                bc0 = bc1;
                f0 = f1;
            }
        }

        // D layout: lane holds column lane % 32; element i is row 8 (i / 4) + 4 h + i % 4
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            const std::int64_t col = n0 + 32 * t + m;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const std::uint32_t r = rb * 32u + 8u * (i / 4) + 4u * static_cast<std::uint32_t>(h) + (i % 4);
                if (r < a.rows)
                    a.out[static_cast<std::int64_t>(r) * a.out_ld + col] =
                        a.ep.active ? epilogue_value(a.ep, acc[t][i], r, col) : acc[t][i];
            }
        }
    }
}

// The same product with each slot's operands staged through LDS (W 16-byte aligned with a row
// stride of whole 16-byte units, scales present, and offsets under the per-gene policy):
// loading a W tile as one 4-byte value per lane and product (32 vector loads per slot and
// wave) cost 37% of the kernel above, and selecting each K step's metadata with four
// readlanes another 10%. Per valid slot, wave w's W tile (the block column's 32 genes x its 64
// columns, 8 KB) and the slot's 32 scales and offsets go straight from memory into a per-wave
// LDS double buffer (8 + 2 loads per lane, no registers); the B operands are then one
// ds_read2_b32 per K step (both column tiles) and the metadata one ds_read2_b32 (scale,
// offset of gene 2kk + h). Genes past `cols` lie outside the loads' descriptors and read as 0
// (their products are 0); in a block column that crosses `cols` the decoded value is also
// set to 0 there, as above. The row block's slot ids are read once (one per lane) and the
// valid ones walked by ballot. kBufs = 2: the next slot's loads are issued while the
// current one's matrix instructions run (68 KB of LDS, two workgroups per CU); kBufs = 1:
// each slot loads, then multiplies (34 KB, four workgroups per CU), and the other waves of
// the SIMD cover the wait -- 3% faster at C4's quantized projection, so the launch takes it.
// Same values and products as the kernel above, same order.
template<int kBits, int kPolicy, int kBufs>
__global__ __launch_bounds__(256) void bell_spmm_quant_lds(BellArgs a, std::int64_t n) {
    constexpr int kTiles = 2;  // 64 output columns per wave and chunk
    constexpr bool kOffsets = kPolicy == CX_DECODE_PER_GENE_AFFINE;
    __shared__ __attribute__((aligned(16))) float wtile[4][kBufs][32 * 64];
    __shared__ __attribute__((aligned(16))) float wmeta[4][kBufs][2 * kWave];  // scales at [0, 64), offsets at [64, 128)
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const std::uint32_t row_blocks = (a.rows + 31u) / 32u;
    const std::uint32_t slot = xcd_major(blockIdx.x, gridDim.x);
    const std::uint32_t rb = a.rb_order != nullptr ? a.rb_order[slot] : slot;
    if (rb >= row_blocks) return;
    const std::uint32_t width = a.ell_cols / 32u;
    const std::uint32_t *slots = a.block_col_idx + static_cast<std::uint64_t>(rb) * width;
    const int m = lane % 32;
    const int h = lane / 32;
    const std::uint32_t row = rb * 32u + static_cast<std::uint32_t>(m);
    const std::uint32_t block_rows = min(32u, a.rows - rb * 32u);
    const rsrc_t rc = make_rsrc(a.packed + static_cast<std::uint64_t>(rb) * 32u * a.row_stride_bytes,
                                block_rows * a.row_stride_bytes);
    const std::uint32_t code_lane = static_cast<std::uint32_t>(m) * a.row_stride_bytes;
    const float row_offset = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET && row < a.rows ? a.row_offsets[row] : 0.0f;
    const float *w = static_cast<const float *>(a.rhs);
    const std::uint32_t row_bytes = static_cast<std::uint32_t>(a.rhs_ld) * 4u;

    for (std::int64_t n0 = static_cast<std::int64_t>(wave) * 64; n0 < n; n0 += 256) {
        // slot s (block column bc): this lane's codes, and the W tile and metadata into buffer buf
        auto load_slot = [&](std::uint32_t (&codes)[kBits], std::uint32_t s, std::uint32_t bc, int buf) {
            const std::uint32_t co = code_lane + s * static_cast<std::uint32_t>(kBits) * 4u;
            if constexpr (kBits >= 4) {
#pragma unroll
                for (int q = 0; q < kBits / 4; ++q) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rc, static_cast<int>(co) + 16 * q, 0, 0);
                    codes[4 * q] = v[0]; codes[4 * q + 1] = v[1]; codes[4 * q + 2] = v[2]; codes[4 * q + 3] = v[3];
                }
            } else {
#pragma unroll
                for (int q = 0; q < kBits; ++q)
                    codes[q] = static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rc, static_cast<int>(co) + 4 * q, 0, 0));
            }
            const std::uint32_t g0 = bc * 32u;
            const std::uint32_t genes = g0 < a.cols ? min(32u, a.cols - g0) : 0u;
            // W: load q covers genes 4q .. 4q + 3, lane l's 16 bytes at gene 4q + l / 16, columns n0 + 4 (l % 16)
            const rsrc_t rw = make_rsrc(w + static_cast<std::int64_t>(g0) * a.rhs_ld, genes * row_bytes);
            const std::uint32_t lane_off = static_cast<std::uint32_t>(lane / 16) * row_bytes
                + static_cast<std::uint32_t>(n0 + 4 * (lane % 16)) * 4u;
#pragma unroll
            for (int q = 0; q < 8; ++q)
                load_lds16(rw, reinterpret_cast<uint4 *>(&wtile[wave][buf][q * 256]), lane_off + 4u * row_bytes * q, 0u);
            // metadata: lane l's 4 bytes = scale (offset) of gene l % 32, the upper half repeating it
            const rsrc_t rs = make_rsrc(a.scales + g0, genes * 4u);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void)&wmeta[wave][buf][0], 4,
                                                     static_cast<std::uint32_t>(m) * 4u, 0, 0, 0);
            if constexpr (kOffsets) {
                const rsrc_t ro = make_rsrc(a.offsets + g0, genes * 4u);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ro, (lds_void)&wmeta[wave][buf][kWave], 4,
                                                         static_cast<std::uint32_t>(m) * 4u, 0, 0, 0);
            }
        };

        cx_floatx16 acc[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;

        auto mfma_slot = [&](const std::uint32_t (&codes)[kBits], std::uint32_t bc, int buf, auto crosses) {
            const float *wt = &wtile[wave][buf][h * 64 + m];
            const float *mt = &wmeta[wave][buf][h];
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                // gene 2kk + h of the block: its code in this lane's row, its (scale, offset) and
                // its W row (columns m and 32 + m of the wave's 64) from LDS
                const int bit = (2 * kk) * kBits;
                const std::uint32_t code = (codes[bit / 32] >> ((bit % 32) + h * kBits)) & ((1u << kBits) - 1u);
                const float scale = mt[2 * kk];
                const float offset = kOffsets ? mt[kWave + 2 * kk] : row_offset;
                float x = __builtin_fmaf(static_cast<float>(code), scale, offset);
                if constexpr (decltype(crosses)::value)
                    x = bc * 32u + static_cast<std::uint32_t>(2 * kk + h) < a.cols ? x : 0.0f;
                const float b0 = wt[kk * 128], b1 = wt[kk * 128 + 32];
                acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, b0, acc[0], 0, 0, 0);
                acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, b1, acc[1], 0, 0, 0);
            }
        };
        auto run_slot = [&](const std::uint32_t (&codes)[kBits], std::uint32_t bc, int buf) {
            if (bc * 32u + 32u <= a.cols) mfma_slot(codes, bc, buf, std::false_type{});
            else mfma_slot(codes, bc, buf, std::true_type{});
        };

        int buf = 0;
        for (std::uint32_t base = 0; base < width; base += kWave) {
            const std::uint32_t cnt = min(static_cast<std::uint32_t>(kWave), width - base);
            const std::uint32_t sid = static_cast<std::uint32_t>(lane) < cnt ? slots[base + lane] : kInvalidBlock;
            unsigned long long valid = __ballot(sid != kInvalidBlock);
            if (valid == 0ull) continue;
            std::uint32_t s = static_cast<std::uint32_t>(__builtin_ctzll(valid));
            std::uint32_t bc0 = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(sid), static_cast<int>(s)));
            std::uint32_t c0[kBits], c1[kBits];
            load_slot(c0, base + s, bc0, buf);
            valid &= valid - 1ull;
            if constexpr (kBufs == 1) {
                // one buffer: each slot's loads, then its products (the other waves of the
                // SIMD cover the wait)
                for (;;) {
                    __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));
                    __builtin_amdgcn_sched_barrier(0);
                    run_slot(c0, bc0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    if (valid == 0ull) break;
                    s = static_cast<std::uint32_t>(__builtin_ctzll(valid));
                    bc0 = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(sid), static_cast<int>(s)));
                    load_slot(c0, base + s, bc0, 0);
                    valid &= valid - 1ull;
                }
                (void)c1;
            } else {
            for (;;) {
                const bool more = valid != 0ull;
                std::uint32_t bc1 = bc0;
                // the current slot's W tile and metadata are in LDS once every earlier load is
                // done; the other buffer's reads were consumed by the previous slot's products
                __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));
                if (more) {
                    s = static_cast<std::uint32_t>(__builtin_ctzll(valid));
                    bc1 = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(sid), static_cast<int>(s)));
                    load_slot(c1, base + s, bc1, buf ^ 1);
                    valid &= valid - 1ull;
                }
                __builtin_amdgcn_sched_barrier(0);
                run_slot(c0, bc0, buf);
                __builtin_amdgcn_sched_barrier(0);
                buf ^= 1;
                if (!more) break;
                bc0 = bc1;
#pragma unroll
                for (int q = 0; q < kBits; ++q) c0[q] = c1[q];
            }
            }
        }

        // D layout: lane holds column lane % 32; element i is row 8 (i / 4) + 4 h + i % 4
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            const std::int64_t col = n0 + 32 * t + m;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const std::uint32_t r = rb * 32u + 8u * (i / 4) + 4u * static_cast<std::uint32_t>(h) + (i % 4);
                if (r < a.rows)
                    a.out[static_cast<std::int64_t>(r) * a.out_ld + col] =
                        a.ep.active ? epilogue_value(a.ep, acc[t][i], r, col) : acc[t][i];
            }
        }
    }
}

int validate_bell(const cx_bell_matrix *m, const void *rhs, std::int64_t rhs_ld,
                  std::int64_t out_cols, const float *out, std::int64_t out_ld) {
    if (m == nullptr || rhs == nullptr || out == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "Blocked-ELL: null matrix, rhs or output");
    if (out_cols <= 0 || out_ld < out_cols || rhs_ld < out_cols)
        return fail(CX_STATUS_INVALID_SHAPE, "Blocked-ELL: bad output columns or leading dimension");
    if (m->block_size == 0u || m->ell_cols == 0u || m->ell_cols % m->block_size != 0u)
        return fail(CX_STATUS_INVALID_SHAPE, "Blocked-ELL: ell_cols must be a positive multiple of block_size");
    if (m->rows != 0u && m->block_col_idx == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "Blocked-ELL: null block_col_idx");
    if ((m->value_layout_flags & ~CX_BELL_BLOCK_MAJOR_VALUES) != 0u || m->reserved != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "Blocked-ELL: unknown value layout flags");
    if (m->bits != 0u && m->value_layout_flags != 0u)
        return fail(CX_STATUS_UNSUPPORTED, "Blocked-ELL: quantized values are row-major only");
    if (m->bits != 0u) {
        if (!(m->bits == 1u || m->bits == 2u || m->bits == 4u || m->bits == 8u))
            return fail(CX_STATUS_UNSUPPORTED, "quantized Blocked-ELL bits must be 1, 2, 4 or 8");
        if (m->row_stride_bytes == 0u || m->packed_values == nullptr)
            return fail(CX_STATUS_INVALID_ARGUMENT, "quantized Blocked-ELL needs packed values and a row stride");
        if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE && m->column_scales == nullptr)
            return fail(CX_STATUS_INVALID_ARGUMENT, "per-gene affine decode needs column scales");
        if (m->decode_policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET && m->row_offsets == nullptr)
            return fail(CX_STATUS_INVALID_ARGUMENT, "column-scale/row-offset decode needs row offsets");
        if (m->decode_policy != CX_DECODE_PER_GENE_AFFINE
            && m->decode_policy != CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
            return fail(CX_STATUS_UNSUPPORTED, "unknown Blocked-ELL decode policy");
    } else {
        if (m->values == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "Blocked-ELL: null values");
        if (m->value_dtype != CELLERATOR_DTYPE_BF16 && m->value_dtype != CELLERATOR_DTYPE_F16
            && m->value_dtype != CELLERATOR_DTYPE_F32)
            return fail(CX_STATUS_UNSUPPORTED, "Blocked-ELL values must be BF16, F16 or F32");
    }
    return CX_STATUS_SUCCESS;
}

BellArgs make_args(const cx_bell_matrix *m, const void *rhs, std::int64_t rhs_ld, float *out,
                   std::int64_t out_ld, const Epilogue &ep) {
    BellArgs a{};
    a.ep = ep;
    a.block_col_idx = m->block_col_idx;
    a.values = m->values;
    a.packed = m->packed_values;
    a.scales = m->column_scales;
    a.offsets = m->column_offsets;
    a.row_offsets = m->row_offsets;
    a.rhs = rhs;
    a.rhs_ld = rhs_ld;
    a.out = out;
    a.out_ld = out_ld;
    a.rows = m->rows;
    a.cols = m->cols;
    a.block_size = m->block_size;
    a.ell_cols = m->ell_cols;
    a.row_stride_bytes = m->row_stride_bytes;
    a.block_major = m->value_layout_flags & CX_BELL_BLOCK_MAJOR_VALUES;
    const std::uint32_t size = m->value_dtype == CELLERATOR_DTYPE_F32 ? 4u : 2u;
    a.a_row_bytes = (a.block_major ? m->block_size : m->ell_cols) * size;
    a.a_slot_bytes = m->block_size * (a.block_major ? m->block_size : 1u) * size;
    a.rb_order = nullptr;
    return a;
}

} // namespace
} // namespace cx

extern "C" int cx_bell_spmm_fwd(const cx_bell_matrix *m, const void *rhs, uint32_t rhs_dtype,
                                int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                                void *stream) {
    return cx_bell_spmm_fwd_epilogue(m, rhs, rhs_dtype, rhs_ld, out_cols, out, out_ld, nullptr,
                                     stream);
}

namespace {

int bell_spmm_fwd_impl(const cx_bell_matrix *m, const void *rhs, uint32_t rhs_dtype, int64_t rhs_ld,
                       int64_t out_cols, float *out, int64_t out_ld, const cx_spmm_epilogue *epilogue,
                       const std::uint32_t *rb_order, void *stream);

} // namespace

extern "C" int cx_bell_spmm_fwd_epilogue(const cx_bell_matrix *m, const void *rhs,
                                         uint32_t rhs_dtype, int64_t rhs_ld, int64_t out_cols,
                                         float *out, int64_t out_ld,
                                         const cx_spmm_epilogue *epilogue, void *stream) {
    return bell_spmm_fwd_impl(m, rhs, rhs_dtype, rhs_ld, out_cols, out, out_ld, epilogue, nullptr, stream);
}

extern "C" int cx_bell_spmm_fwd_ordered(const cx_bell_matrix *m, const void *rhs, uint32_t rhs_dtype,
                                        int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                                        const uint32_t *row_block_order, void *stream) {
    cx::clear_error();
    if (row_block_order == nullptr && m != nullptr && m->rows != 0u)
        return cx::fail(CX_STATUS_INVALID_ARGUMENT, "cx_bell_spmm_fwd_ordered: null row-block order");
    return bell_spmm_fwd_impl(m, rhs, rhs_dtype, rhs_ld, out_cols, out, out_ld, nullptr, row_block_order, stream);
}

namespace {

int bell_spmm_fwd_impl(const cx_bell_matrix *m, const void *rhs, uint32_t rhs_dtype, int64_t rhs_ld,
                       int64_t out_cols, float *out, int64_t out_ld, const cx_spmm_epilogue *epilogue,
                       const std::uint32_t *rb_order, void *stream) {
    using namespace cx;
    clear_error();
    int rc = validate_bell(m, rhs, rhs_ld, out_cols, out, out_ld);
    if (rc != CX_STATUS_SUCCESS) return rc;
    Epilogue ep;
    rc = make_epilogue(epilogue, m->rows, out_cols, out, out_ld, &ep, "cx_bell_spmm_fwd");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (rhs_dtype != CELLERATOR_DTYPE_F32 && rhs_dtype != CELLERATOR_DTYPE_F16
        && rhs_dtype != CELLERATOR_DTYPE_BF16)
        return fail(CX_STATUS_UNSUPPORTED, "Blocked-ELL rhs must be F32, F16 or BF16");
    if (m->rows == 0u) return CX_STATUS_SUCCESS;
    BellArgs a = make_args(m, rhs, rhs_ld, out, out_ld, ep);
    a.rb_order = rb_order;
    if (m->bits != 0u && m->block_size == 32u && rhs_dtype == CELLERATOR_DTYPE_F32 && out_cols % 64 == 0
        && m->row_stride_bytes % 4u == 0u && m->row_stride_bytes >= m->ell_cols * m->bits / 8u
        && static_cast<std::uint64_t>(m->row_stride_bytes) * 32u <= 0xffffffffull) {
        // the matrix-core form (same values, fp32 products and sums in another order); operands
        // through LDS when W's rows are whole 16-byte units and 32 of them span under 4 GiB
        const hipStream_t s = static_cast<hipStream_t>(stream);
        const dim3 grid((m->rows + 31u) / 32u), block(256);
        const bool lds_w = (reinterpret_cast<std::uintptr_t>(rhs) & 15u) == 0u && rhs_ld % 4 == 0
            && static_cast<std::uint64_t>(rhs_ld) * 4u * 32u <= 0xffffffffull && m->column_scales != nullptr
            && (m->decode_policy != CX_DECODE_PER_GENE_AFFINE || m->column_offsets != nullptr);
#define CX_QBELL_W(B, P)                                                                                 \
    do {                                                                                                 \
        if (lds_w) hipLaunchKernelGGL((bell_spmm_quant_lds<B, P, 1>), grid, block, 0, s, a, out_cols);       \
        else hipLaunchKernelGGL((bell_spmm_quant_mfma<B, P>), grid, block, 0, s, a, out_cols);              \
    } while (0)
#define CX_QBELL(B)                                                                                      \
    do {                                                                                                 \
        if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE) CX_QBELL_W(B, CX_DECODE_PER_GENE_AFFINE);       \
        else CX_QBELL_W(B, CX_DECODE_COLUMN_SCALE_ROW_OFFSET);                                           \
    } while (0)
        switch (m->bits) {
        case 1: CX_QBELL(1); break;
        case 2: CX_QBELL(2); break;
        case 4: CX_QBELL(4); break;
        default: CX_QBELL(8); break;
        }
#undef CX_QBELL
#undef CX_QBELL_W
        return check_launch("bell_spmm_quant_mfma");
    }
    // the per-element kernel walks rows in matrix order (no row-block order)
    const std::uint64_t threads = static_cast<std::uint64_t>(m->rows) * kWave;
    hipLaunchKernelGGL(bell_spmm_generic, dim3(static_cast<unsigned>((threads + 255) / 256)),
                       dim3(256), 0, static_cast<hipStream_t>(stream), a, m->value_dtype,
                       rhs_dtype, m->bits, m->decode_policy, out_cols);
    return check_launch("bell_spmm_generic");
}

} // namespace

extern "C" int cx_bell_pack_rhs(const uint16_t *rhs_bf16, int64_t rhs_ld, uint32_t k, uint32_t n,
                                uint16_t *packed, void *stream) {
    using namespace cx;
    clear_error();
    if (rhs_bf16 == nullptr || packed == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_bell_pack_rhs: null rhs or packed output");
    if (k == 0u || n == 0u || n % 32u != 0u || rhs_ld < static_cast<int64_t>(n))
        return fail(CX_STATUS_INVALID_SHAPE, "cx_bell_pack_rhs: bad shape (n must be a multiple of 32)");
    const std::uint64_t total = static_cast<std::uint64_t>((k + 31u) / 32u) * n * 32u;
    hipLaunchKernelGGL(pack_rhs_frag_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256),
                       0, static_cast<hipStream_t>(stream), rhs_bf16, rhs_ld, k, n, packed);
    return check_launch("cx_bell_pack_rhs");
}

namespace cx {
int pack_panel_columns(const std::uint16_t *rhs, std::int64_t rhs_ld, std::uint32_t k, std::uint32_t n,
                       std::uint16_t *packed, hipStream_t stream) {
    const std::uint64_t total = static_cast<std::uint64_t>((k + 31u) / 32u) * n * 32u;
    hipLaunchKernelGGL(pack_rhs_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256),
                       0, stream, rhs, rhs_ld, k, n, packed);
    return check_launch("pack_rhs_kernel");
}
} // namespace cx

extern "C" int cx_bell_block_major_values(const cx_bell_matrix *m, void *out, uint64_t capacity,
                                          void *stream) {
    using namespace cx;
    clear_error();
    if (m == nullptr || out == nullptr || (m->rows != 0u && m->values == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_bell_block_major_values: null matrix, values or output");
    if (m->bits != 0u || m->value_layout_flags != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_bell_block_major_values: needs row-major unquantized values");
    if (m->block_size == 0u || m->ell_cols == 0u || m->ell_cols % m->block_size != 0u)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_bell_block_major_values: ell_cols must be a positive multiple of block_size");
    const std::uint32_t size = m->value_dtype == CELLERATOR_DTYPE_F32 ? 4u
        : (m->value_dtype == CELLERATOR_DTYPE_BF16 || m->value_dtype == CELLERATOR_DTYPE_F16) ? 2u : 0u;
    if (size == 0u) return fail(CX_STATUS_UNSUPPORTED, "cx_bell_block_major_values: values must be BF16, F16 or F32");
    const std::uint64_t total = static_cast<std::uint64_t>((m->rows + m->block_size - 1u) / m->block_size)
        * m->ell_cols * m->block_size;
    if (capacity < total * size)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_bell_block_major_values: output capacity is too small");
    if (total == 0u) return CX_STATUS_SUCCESS;
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (size == 4u)
        hipLaunchKernelGGL(block_major_kernel<std::uint32_t>, grid, dim3(256), 0, s,
                           static_cast<const std::uint32_t *>(m->values), m->rows, m->block_size, m->ell_cols,
                           total, static_cast<std::uint32_t *>(out));
    else
        hipLaunchKernelGGL(block_major_kernel<std::uint16_t>, grid, dim3(256), 0, s,
                           static_cast<const std::uint16_t *>(m->values), m->rows, m->block_size, m->ell_cols,
                           total, static_cast<std::uint16_t *>(out));
    return check_launch("cx_bell_block_major_values");
}

extern "C" int cx_bell_spmm_fwd_packed(const cx_bell_matrix *m, const uint16_t *packed_rhs,
                                       int64_t out_cols, float *out, int64_t out_ld,
                                       void *stream) {
    return cx_bell_spmm_fwd_packed_epilogue(m, packed_rhs, out_cols, out, out_ld, nullptr, stream);
}

extern "C" int cx_bell_spmm_fwd_packed_epilogue(const cx_bell_matrix *m,
                                                const uint16_t *packed_rhs, int64_t out_cols,
                                                float *out, int64_t out_ld,
                                                const cx_spmm_epilogue *epilogue, void *stream) {
    using namespace cx;
    clear_error();
    int rc = validate_bell(m, packed_rhs, out_cols, out_cols, out, out_ld);
    if (rc != CX_STATUS_SUCCESS) return rc;
    Epilogue ep;
    rc = make_epilogue(epilogue, m->rows, out_cols, out, out_ld, &ep, "cx_bell_spmm_fwd_packed");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (m->bits != 0u || m->value_dtype != CELLERATOR_DTYPE_BF16 || m->block_size != 32u)
        return fail(CX_STATUS_UNSUPPORTED,
                    "MFMA Blocked-ELL needs unquantized BF16 values and 32x32 blocks");
    if (out_cols != 64 && out_cols != 128 && out_cols != 256)
        return fail(CX_STATUS_UNSUPPORTED, "MFMA Blocked-ELL supports 64, 128 or 256 output columns");
    if ((reinterpret_cast<std::uintptr_t>(m->values) & 15u) != 0u
        || (reinterpret_cast<std::uintptr_t>(packed_rhs) & 15u) != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "MFMA Blocked-ELL operands must be 16-byte aligned");
    if (m->rows == 0u) return CX_STATUS_SUCCESS;
    const BellArgs a = make_args(m, packed_rhs, out_cols, out, out_ld, ep);
    const unsigned row_blocks = (m->rows + 31u) / 32u;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const std::uint64_t panel = static_cast<std::uint64_t>((m->cols + 31u) / 32u) * static_cast<std::uint64_t>(out_cols) * 64u;
    const std::uint64_t block_rows = static_cast<std::uint64_t>(32u) * m->ell_cols * 2u;
    if (panel > 0xFFFFFFFFull || block_rows > 0xFFFFFFFFull)
        return fail(CX_STATUS_INVALID_SHAPE, "MFMA Blocked-ELL: packed panel or row block exceeds 4 GiB");
    const std::uint32_t pb = static_cast<std::uint32_t>(panel);
    const std::uint32_t *none = nullptr;
    switch (out_cols) {
    case 64: hipLaunchKernelGGL(bell_spmm_mfma<64>, dim3(row_blocks), dim3(64), 0, s, a, packed_rhs, pb, none); break;
    case 128: hipLaunchKernelGGL(bell_spmm_mfma<128>, dim3(row_blocks), dim3(128), 0, s, a, packed_rhs, pb, none); break;
    default: hipLaunchKernelGGL(bell_spmm_mfma<256>, dim3(row_blocks), dim3(256), 0, s, a, packed_rhs, pb, none); break;
    }
    return check_launch("bell_spmm_mfma");
}

extern "C" int cx_bell_spmm_fwd_grouped(const cx_bell_matrix *m, const uint16_t *packed_rhs,
                                        const cx_bell_groups *groups, int64_t out_cols,
                                        float *out, int64_t out_ld, void *stream) {
    return cx_bell_spmm_fwd_grouped_epilogue(m, packed_rhs, groups, out_cols, out, out_ld, nullptr,
                                             stream);
}

extern "C" int cx_bell_spmm_fwd_grouped_epilogue(const cx_bell_matrix *m,
                                                 const uint16_t *packed_rhs,
                                                 const cx_bell_groups *groups, int64_t out_cols,
                                                 float *out, int64_t out_ld,
                                                 const cx_spmm_epilogue *epilogue, void *stream) {
    using namespace cx;
    clear_error();
    int rc = validate_bell(m, packed_rhs, out_cols, out_cols, out, out_ld);
    if (rc != CX_STATUS_SUCCESS) return rc;
    Epilogue ep;
    rc = make_epilogue(epilogue, m->rows, out_cols, out, out_ld, &ep, "cx_bell_spmm_fwd_grouped");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (groups == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "grouped Blocked-ELL: null groups");
    if (m->bits != 0u || m->value_dtype != CELLERATOR_DTYPE_BF16 || m->block_size != 32u)
        return fail(CX_STATUS_UNSUPPORTED,
                    "MFMA Blocked-ELL needs unquantized BF16 values and 32x32 blocks");
    if (out_cols != 64 && out_cols != 128 && out_cols != 256)
        return fail(CX_STATUS_UNSUPPORTED, "MFMA Blocked-ELL supports 64, 128 or 256 output columns");
    if ((reinterpret_cast<std::uintptr_t>(m->values) & 15u) != 0u
        || (reinterpret_cast<std::uintptr_t>(packed_rhs) & 15u) != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "MFMA Blocked-ELL operands must be 16-byte aligned");
    const std::uint32_t row_blocks = (m->rows + 31u) / 32u;
    if (static_cast<std::uint64_t>(groups->grouped_row_blocks) + groups->single_count != row_blocks
        || (groups->group_count != 0u
            && (groups->group_offsets == nullptr || groups->grouped_row_blocks < groups->group_count
                || groups->grouped_row_blocks > 4ull * groups->group_count))
        || (row_blocks != 0u && groups->order == nullptr))
        return fail(CX_STATUS_INVALID_SHAPE, "grouped Blocked-ELL: groups do not cover the row blocks");
    if (m->ell_cols / 32u > 64u)
        return fail(CX_STATUS_UNSUPPORTED, "grouped Blocked-ELL supports at most 64 slots per row block");
    if (m->rows == 0u) return CX_STATUS_SUCCESS;
    const BellArgs a = make_args(m, packed_rhs, out_cols, out, out_ld, ep);
    const std::uint64_t panel = static_cast<std::uint64_t>((m->cols + 31u) / 32u) * static_cast<std::uint64_t>(out_cols) * 64u;
    if (panel > 0xFFFFFFFFull || static_cast<std::uint64_t>(32u) * m->ell_cols * 2u > 0xFFFFFFFFull)
        return fail(CX_STATUS_INVALID_SHAPE, "MFMA Blocked-ELL: packed panel or row block exceeds 4 GiB");
    const std::uint32_t pb = static_cast<std::uint32_t>(panel);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 gblock(kWave * kGroupWaves);
    const dim3 ggrid(groups->group_count + groups->single_count);
    const std::uint32_t gc = groups->group_count, grb = groups->grouped_row_blocks;
    switch (out_cols) {
    case 64: hipLaunchKernelGGL(bell_spmm_mfma_grouped<64>, ggrid, gblock, 0, s, a, packed_rhs, pb, groups->order, groups->group_offsets, gc, grb); break;
    case 128:
        if (a.block_major) hipLaunchKernelGGL((bell_spmm_mfma_slab<128, true, 4>), ggrid, gblock, 0, s, a, packed_rhs, pb, groups->order, groups->group_offsets, gc, grb);
        else hipLaunchKernelGGL((bell_spmm_mfma_slab<128, false, 4>), ggrid, gblock, 0, s, a, packed_rhs, pb, groups->order, groups->group_offsets, gc, grb);
        break;
    default: {
        const dim3 gblock8(kWave * 8);
        if (a.block_major) hipLaunchKernelGGL((bell_spmm_mfma_slab<256, true, 8>), ggrid, gblock8, 0, s, a, packed_rhs, pb, groups->order, groups->group_offsets, gc, grb);
        else hipLaunchKernelGGL((bell_spmm_mfma_slab<256, false, 8>), ggrid, gblock8, 0, s, a, packed_rhs, pb, groups->order, groups->group_offsets, gc, grb);
        break;
    }
    }
    rc = check_launch("bell_spmm_mfma_grouped");
    return rc;
}
