// qcsr_parts.hip -- quantized CSR SpMM with the weight panel streamed through LDS by gene
// part (fp16 weights, N a multiple of 64 in blocks of 64 columns), and the gradient of the
// stored values by the same part walk.
//
// Same value semantics as qcsr_spmm.hip (decode fma(float(code), scale, offset), exact fp16
// widening, fp32 products and sums); only the summation order differs, and it is fixed.
//
// Why: gathering a 128-byte weight row per nonzero through the texture path, plus an
// 8-byte metadata gather per code, keeps the row-wave kernel far below HBM speed. LDS
// serves the same 16-byte-per-lane gathers at about twice the rate, and the per-gene
// metadata of a part sits beside its weight rows.
//
// One workgroup of 16 waves per CU (LDS-bound) walks the genes in parts of kPartGenes. Each
// part's fp16 weight rows (128 B each) and (scale, offset) pairs are copied into LDS by
// buffer loads that write LDS directly; then every wave works through its rows' entries in
// that part, and the next part replaces it. A prologue ranks the block's rows by length so
// every wave carries about the same number of nonzeros into each part barrier.
//
// Forward (qcsr_spmm_groups): lane group g (8 lanes) of a wave owns one row of each of the
// wave's layers, and lane j of the group holds that row's output columns 8j..8j+7 in
// registers, so a row costs 8 registers and a workgroup owns 512 rows (details at the
// kernel). Backward values (qcsr_bwd_values_groups) use the same walk with the row's
// gradient in place of the output sums.
#include "qcsr_common.hpp"

namespace cx {
namespace {

constexpr int kPartGenes = 1024;                 // 128 KB of fp16 weight rows per part
constexpr std::uint32_t kNoRow = 0xffffffffu;

using rsrc_t = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, std::uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

using lds_ptr = __attribute__((address_space(3))) void *;

// The fp16 weight rows of genes [lo, hi) straight from memory into LDS (buffer loads with
// the lds flag: wave instruction k of wave w fills 1 KB, 8 rows, at no register cost);
// loads past the part's last row return zeros.
template<int kWaves>
__device__ __forceinline__ void load_part_weights(uint4 *w, const std::uint16_t *rhs, std::int64_t rhs_ld,
                                                  int lo, int hi, int wave, int lane) {
    constexpr int kChunks = kPartGenes * 8 / kWave;  // 1 KB wave loads per part
    static_assert(kChunks % kWaves == 0, "part chunks must divide among the waves");
    const std::uint32_t row_bytes = static_cast<std::uint32_t>(rhs_ld) * 2u;
    // One descriptor per chunk (built in scalar registers) and one lane offset for all of
    // them, so the copy keeps a single address register live across the part loop.
    const std::uint32_t lane_off = static_cast<std::uint32_t>(lane >> 3) * row_bytes + static_cast<std::uint32_t>(lane & 7) * 16u;
#pragma unroll
    for (int k = 0; k < kChunks / kWaves; ++k) {
        const int chunk = k * kWaves + wave;
        const int row0 = chunk * 8;  // first of the chunk's 8 rows within the part
        const int left = hi - lo - row0;
        const rsrc_t rw = make_rsrc(rhs + static_cast<std::int64_t>(lo + row0) * rhs_ld,
                                    left > 0 ? static_cast<std::uint32_t>(left - 1) * row_bytes + 128u : 0u);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr)(&w[chunk * kWave]), 16, lane_off, 0, 0, 0);
    }
}

// The weight rows and (scale, offset) pairs of genes [lo, hi) into LDS. Interleaved pairs
// go straight to LDS like the weights; the other decode policies build them in registers.
// kWait: wait for every load in flight (vmcnt 0) before returning; otherwise the caller waits.
template<int kPolicy, int kWaves, typename Shared, bool kWait = true>
__device__ __forceinline__ void load_part(Shared &sh, const QcsrArgs &a, int lo, int hi, int wave, int lane,
                                          int tid) {
    const int span = hi - lo;
    load_part_weights<kWaves>(sh.w, static_cast<const std::uint16_t *>(a.rhs), a.rhs_ld, lo, hi, wave, lane);
    if constexpr (kPolicy == CX_DECODE_PER_GENE_AFFINE_PAIRS) {
        constexpr int kMetaChunks = kPartGenes * 8 / (kWave * 16);  // 2 pairs per lane
        if (wave < kMetaChunks) {
            const int left = span - wave * 2 * kWave;  // pairs of this wave's chunk
            const rsrc_t rm = make_rsrc(reinterpret_cast<const float2 *>(a.scales) + lo + wave * 2 * kWave,
                                        left > 0 ? static_cast<std::uint32_t>(left) * 8u : 0u);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_ptr)(&sh.meta[wave * 2 * kWave]), 16,
                                                     static_cast<std::uint32_t>(lane) * 16u, 0, 0, 0);
        }
    } else {
        for (int g = tid; g < span; g += kWaves * kWave) {
            float2 md;
            md.x = a.scales != nullptr ? a.scales[lo + g] : 1.0f;
            md.y = kPolicy == CX_DECODE_PER_GENE_AFFINE && a.offsets != nullptr ? a.offsets[lo + g] : 0.0f;
            sh.meta[g] = md;
        }
    }
    if constexpr (kWait) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the LDS writes of the loads above
}

__device__ __forceinline__ void fma8(float (&p)[8], float x, uint4 w) {
    const std::uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        p[2 * k] = __builtin_fmaf(x, h2f(static_cast<std::uint16_t>(words[k] & 0xffffu)), p[2 * k]);
        p[2 * k + 1] = __builtin_fmaf(x, h2f(static_cast<std::uint16_t>(words[k] >> 16)), p[2 * k + 1]);
    }
}

// Plain per-row path for rows the part walk could not finish: lane c accumulates column
// c over the row's entries in storage order; columns outside [0, cols) contribute nothing.
// In the hybrid tail the walk starts at row_start[row] from the head's partial sum.
// The head's sums of `row`, columns 8j .. 8j + 7: its partials added in order.
__device__ __forceinline__ void head_init8(const QcsrArgs &a, std::uint32_t row, int j, float *acc) {
    const float *p = a.acc_init + static_cast<std::int64_t>(row) * 64 + 8 * j;
    float4 i0 = reinterpret_cast<const float4 *>(p)[0], i1 = reinterpret_cast<const float4 *>(p)[1];
    for (std::uint32_t k = 1; k < a.acc_parts; ++k) {
        const float4 *q = reinterpret_cast<const float4 *>(p + k * a.acc_part_stride);
        const float4 u0 = q[0], u1 = q[1];
        i0.x += u0.x; i0.y += u0.y; i0.z += u0.z; i0.w += u0.w;
        i1.x += u1.x; i1.y += u1.y; i1.z += u1.z; i1.w += u1.w;
    }
    acc[0] = i0.x; acc[1] = i0.y; acc[2] = i0.z; acc[3] = i0.w;
    acc[4] = i1.x; acc[5] = i1.y; acc[6] = i1.z; acc[7] = i1.w;
}

template<int kBits, int kPolicy>
__device__ float row_fallback(const QcsrArgs &a, std::uint32_t row, int lane) {
    const std::int64_t begin = a.row_ptr[row], end = a.row_ptr[row + 1];
    const std::uint8_t *pbase = a.packed + a.packed_row_ptr[row];
    const float row_offset = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET && a.row_offsets != nullptr
        ? a.row_offsets[row] : 0.0f;
    const std::uint16_t *rhs = static_cast<const std::uint16_t *>(a.rhs);
    float acc = 0.0f;
    if (a.acc_init != nullptr)
        for (std::uint32_t k = 0; k < (a.acc_parts > 1u ? a.acc_parts : 1u); ++k)
            acc += a.acc_init[static_cast<std::int64_t>(row) * 64 + lane + k * a.acc_part_stride];
    const std::int64_t start = a.row_start != nullptr ? a.row_start[row] : begin;
    for (std::int64_t i = start; i < end; ++i) {
        const std::uint32_t col = static_cast<std::uint32_t>(a.col_idx[i]);
        if (col >= a.cols) continue;
        int c = 0;
        const float x = load_entry<kBits, kPolicy, ValueMode::quantized>(a, i, begin, pbase, row_offset, c);
        acc = __builtin_fmaf(x, h2f(rhs[static_cast<std::int64_t>(col) * a.rhs_ld + lane]), acc);
    }
    return acc;
}

// ---- row-group form: lane group g of a wave owns one row of every layer ----------------------
//
// Each wave owns kLayers layers of 8 rows. Lane group g (8 lanes) owns row g of every layer,
// and lane j of the group holds columns 8j..8j+7 of that row's output in registers for the
// whole launch (8 fp32 per row and lane; no cross-lane reduction at the end). So the row
// control of a part is vector work over 8 rows at once, and a row costs 8 registers instead
// of 64, which lets one workgroup own 512 rows and copy each part for 4x as many rows.
//
// Every layer keeps a 64-entry window of each of its rows in registers: lane j holds the
// column indices of entries cur + 8j .. cur + 8j + 7 and the two (three for 8-bit codes)
// aligned dwords that hold their codes. A pass over a layer:
//   * counts the window entries with column < hi (entries past the row end excluded): with
//     sorted columns this is the row's run in the part (`run`, at most 64);
//   * decodes the run in four fills of two window slots per lane: slots 2f, 2f + 1 of lane j
//     (entries 8j + 2f, 8j + 2f + 1) go to stage slots 2j, 2j + 1 of the group, so each
//     fill's valid entries are a prefix of the group's 16 stage slots; the rest are pads
//     (the all-zero weight row, value 0);
//   * steps through the fill: lane j of group g reads 16 B of the weight row of the group's
//     staged entry and issues 8 v_fma_mix_f32 into its 8 partial sums, two entries per step;
//   * advances the cursors by the runs and reloads the windows at the new cursors (buffer
//     loads that complete behind the rest of the part); a row whose run filled the whole
//     window continues in another pass.
// An entry inside a run whose column is outside the part (columns out of order across
// parts) marks the row broken; broken rows and rows whose cursor stops before the row end
// (a column outside [0, cols)) are recomputed at the end on the plain per-row path.

constexpr int kPadGene = kPartGenes;  // all-zero weight row, (0, 0) metadata

// Scratch of the prologue that assigns rows to (wave, layer, group) slots.
template<int kWaves, int kLayers>
struct GroupPrologue {
    static constexpr int kRows = kWaves * kLayers * 8;
    int len[kRows];                 // row lengths by position in the block (-1: no row)
    int by_rank[kRows];             // row lengths by rank
    int set_slot[kRows / 8];        // wave * kLayers + layer of row set s
};

template<int kWaves, int kLayers>
struct GroupsShared {
    static constexpr int kRows = kWaves * kLayers * 8;
    union {
        uint4 stage[kWaves][8][9];  // per wave and lane group: 16 (metadata byte offset, value) pairs (+16 B pad)
        GroupPrologue<kWaves, kLayers> pro;
    } u;
    float2 meta[kPartGenes + 2];    // (scale, offset) per gene of the part; [kPadGene] = (0, 0)
    uint4 w[(kPartGenes + 1) * 8];  // fp16 weight rows of the part; row kPadGene is zeros
    std::uint32_t rows[kRows];      // row of (wave, layer, group)
    int qbits[kWaves][kLayers][8];  // code bit offset q of (wave, layer, group): kept here, not in registers
};

// Rank the block's rows by length (descending, ties by index); ranks 8s .. 8s + 7 form row
// set s (similar lengths, so the 8 groups of a layer finish their runs together), and the
// sets go, heaviest first, to the least-loaded wave with a layer left (ties: the lower wave),
// so the waves carry about the same number of nonzeros into every part barrier even when a
// block's longest rows are several times its median.
template<int kWaves, int kLayers>
__device__ __forceinline__ void assign_groups(GroupPrologue<kWaves, kLayers> &pro, std::uint32_t *rows_out,
                                              const std::int32_t *row_ptr, std::uint32_t end_row, std::uint32_t first,
                                              int tid) {
    constexpr int kRows = kWaves * kLayers * 8;
    constexpr int kSets = kRows / 8;
    int *len = pro.len;
    const std::uint32_t row = first + static_cast<std::uint32_t>(tid);  // the block's rows: [first, end_row)
    if (tid < kRows) len[tid] = row < end_row ? row_ptr[row + 1] - row_ptr[row] : -1;
    __syncthreads();
    int rank = 0;
    if (tid < kRows) {
        const int my = len[tid];
        const int4 *l4 = reinterpret_cast<const int4 *>(len);
#pragma unroll 4
        for (int u = 0; u < kRows / 4; ++u) {
            const int4 v = l4[u];
            const int b = 4 * u;
            rank += v.x > my || (v.x == my && b < tid) ? 1 : 0;
            rank += v.y > my || (v.y == my && b + 1 < tid) ? 1 : 0;
            rank += v.z > my || (v.z == my && b + 2 < tid) ? 1 : 0;
            rank += v.w > my || (v.w == my && b + 3 < tid) ? 1 : 0;
        }
        pro.by_rank[rank] = my;
    }
    __syncthreads();
    if (tid < kWave) {
        // One wave deals the sets: lane s holds set s's load, lane w (< kWaves) the load of
        // wave w; per set, a DPP min over lanes 0..15 of (load, lane) finds the least-loaded
        // wave with a layer left. Loads saturate at 2^27 (only the balance depends on them).
        static_assert(kSets <= kWave && kWaves == 16, "one wave deals the sets to 16 waves");
        const int lane = tid;
        std::uint32_t set_load = 0u;
        if (lane < kSets)
            for (int k = 0; k < 8; ++k) {
                const int v = pro.by_rank[lane * 8 + k];
                set_load += static_cast<std::uint32_t>(v > 0 ? min(v, 1 << 20) : 0);
            }
        std::uint32_t wave_load = 0u;
        int used = 0;
        for (int st = 0; st < kSets; ++st) {
            const std::uint32_t load = __builtin_amdgcn_readlane(set_load, st);
            std::uint32_t key = lane < kWaves && used < kLayers ? (min(wave_load, (1u << 27) - 1u) << 4) | lane
                                                                 : 0xffffffffu;
            key = min(key, static_cast<std::uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(key), 0x121, 0xf, 0xf, false)));
            key = min(key, static_cast<std::uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(key), 0x122, 0xf, 0xf, false)));
            key = min(key, static_cast<std::uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(key), 0x124, 0xf, 0xf, false)));
            key = min(key, static_cast<std::uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(key), 0x128, 0xf, 0xf, false)));
            const int best = static_cast<int>(__builtin_amdgcn_readlane(key, 0) & 15u);
            const int layer = __builtin_amdgcn_readlane(used, best);
            if (lane == best) {
                wave_load += load;
                ++used;
            }
            if (lane == 0) pro.set_slot[st] = best * kLayers + layer;
        }
    }
    __syncthreads();
    if (tid < kRows) rows_out[pro.set_slot[rank / 8] * 8 + rank % 8] = row < end_row ? row : kNoRow;
    __syncthreads();
}

// Sum over the 8 lanes of each lane group (integer form of the DPP butterfly).
__device__ __forceinline__ int group_sum8i(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false);
    return v;
}

// Maximum over the wave of a value that is uniform within each lane group.
__device__ __forceinline__ int wave_max_groups(int v) {
    const int r = __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false);  // row_ror:8
    v = v > r ? v : r;
    const auto s = __builtin_amdgcn_permlane16_swap(static_cast<std::uint32_t>(v), static_cast<std::uint32_t>(v),
                                                    false, false);
    v = static_cast<int>(s[0] > s[1] ? s[0] : s[1]);
    const auto t = __builtin_amdgcn_permlane32_swap(static_cast<std::uint32_t>(v), static_cast<std::uint32_t>(v),
                                                    false, false);
    v = static_cast<int>(t[0] > t[1] ? t[0] : t[1]);
    return __builtin_amdgcn_readfirstlane(v);
}

// Entries of fill f (window entries 8j + 2f + r, j < 8, r < 2) below `run`.
__device__ __forceinline__ int fill_count(int run, int f) {
    const int t = run - 2 * f;
    if (t <= 0) return 0;
    const int blocks = t >> 3;
    if (blocks >= 8) return 16;
    const int rem = t & 7;
    return 2 * blocks + (rem < 2 ? rem : 2);
}

template<int kBits, int kPolicy, int kWaves, int kLayers, bool kSorted>
__global__ __launch_bounds__(kWaves * kWave) void qcsr_spmm_groups(QcsrArgs a) {
    using Shared = GroupsShared<kWaves, kLayers>;
    constexpr int kCodeDw = kBits == 8 ? 3 : 2;
    constexpr std::uint32_t kMask = (1u << kBits) - 1u;
    __shared__ Shared sh;
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int grp = lane >> 3;
    const int j = lane & 7;
    // The block's rows: an even share [first, last) of the matrix, at most Shared::kRows (the
    // launch uses at least ceil(rows / Shared::kRows) blocks).
    const std::uint32_t first = static_cast<std::uint32_t>(std::uint64_t{blockIdx.x} * a.rows / gridDim.x);
    const std::uint32_t last = static_cast<std::uint32_t>((std::uint64_t{blockIdx.x} + 1u) * a.rows / gridDim.x);

    if (tid < 8) sh.w[kPadGene * 8 + tid] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 8) sh.meta[kPadGene] = make_float2(0.0f, 0.0f);
    assign_groups<kWaves, kLayers>(sh.u.pro, sh.rows, a.row_ptr, last, first, tid);

    // The block's entries and packed bytes, addressed by 32-bit buffer offsets.
    const int wg_begin = __builtin_amdgcn_readfirstlane(a.row_ptr[first]);
    const int wg_end = __builtin_amdgcn_readfirstlane(a.row_ptr[last]);
    const int pk_al = __builtin_amdgcn_readfirstlane(a.packed_row_ptr[first]) & ~3;
    const int pk_end = __builtin_amdgcn_readfirstlane(a.packed_row_ptr[last]);
    const bool fits = wg_end - wg_begin < (1 << 27);  // bit offsets of the codes stay below 2^31
    // A window reads up to 63 entries (and their code bytes) past the block's last entry:
    // the ranges extend that far where the arrays do. In the block whose ranges stop at an
    // array's end (`tail`), windows that reach past it are reloaded dword by dword and byte
    // by byte, so no valid entry shares a multi-dword load with bytes outside the range.
    const int nnz_all = __builtin_amdgcn_readfirstlane(a.row_ptr[a.rows]);
    const int pk_all = __builtin_amdgcn_readfirstlane(a.packed_row_ptr[a.rows]);
    const int col_n = nnz_all - wg_end < 72 ? nnz_all - wg_begin : wg_end - wg_begin + 72;
    const int pk_n = pk_all - pk_end < 128 ? pk_all - pk_al : pk_end - pk_al + 128;
    const bool tail = nnz_all - wg_end < 72 || pk_all - pk_end < 128;
    const std::uint32_t col_lim = fits ? static_cast<std::uint32_t>(col_n) * 4u : 0u;
    const std::uint32_t pk_lim = fits ? static_cast<std::uint32_t>(pk_n) : 0u;
    const rsrc_t rc = make_rsrc(a.col_idx + wg_begin, col_lim);
    const rsrc_t rp = make_rsrc(a.packed + pk_al, pk_lim);

    // Per layer (values uniform within the lane group): cursor and end relative to the
    // block's first entry, bit offset q of the codes (entry e's code starts at bit
    // q + e * kBits of the block's aligned packed bytes), row offset.
    float acc[kLayers][8];
    std::uint32_t colw[kLayers][8];
    std::uint32_t cw[kLayers][kCodeDw];
    int cur[kLayers], end[kLayers];
    float roff[kLayers];

    // Window of layer l at entry offset e0 = cursor + 8j: column slots 4h..4h+3 (h = 0, 1)
    // and the dwords holding the 8 entries' codes.
    auto load_cols = [&](int l, int h, std::uint32_t e0) {
        const auto c = __builtin_amdgcn_raw_buffer_load_b128(rc, e0 * 4u + 16u * h, 0, 0);
        colw[l][4 * h] = c[0]; colw[l][4 * h + 1] = c[1]; colw[l][4 * h + 2] = c[2]; colw[l][4 * h + 3] = c[3];
    };
    auto load_codes = [&](int l, std::uint32_t e0, int q) {
        const std::uint32_t al = ((static_cast<std::uint32_t>(q) + e0 * kBits) >> 3) & ~3u;
        if constexpr (kCodeDw == 2) {
            const auto c = __builtin_amdgcn_raw_buffer_load_b64(rp, al, 0, 0);
            cw[l][0] = c[0]; cw[l][1] = c[1];
        } else {
            const auto c = __builtin_amdgcn_raw_buffer_load_b96(rp, al, 0, 0);
            cw[l][0] = c[0]; cw[l][1] = c[1]; cw[l][2] = c[2];
        }
    };
    auto load_window = [&](int l, int q) {
        const std::uint32_t e0 = static_cast<std::uint32_t>(cur[l] + 8 * j);
        load_cols(l, 0, e0);
        load_cols(l, 1, e0);
        load_codes(l, e0, q);
    };

    // Tail block only: reload layer l's window with single-dword / single-byte loads when
    // some lane's multi-dword loads reach past the array ends.
    auto fix_tail = [&](int l) {
        const std::uint32_t e0 = static_cast<std::uint32_t>(cur[l] + 8 * j);
        const std::uint32_t al = ((static_cast<std::uint32_t>(sh.qbits[wave][l][grp]) + e0 * kBits) >> 3) & ~3u;
        if (__builtin_amdgcn_ballot_w64(e0 * 4u + 32u > col_lim || al + 4u * kCodeDw > pk_lim) == 0u) return;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            colw[l][k] = static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rc, (e0 + k) * 4u, 0, 0));
#pragma unroll
        for (int d = 0; d < kCodeDw; ++d) {
            std::uint32_t v = 0u;
#pragma unroll
            for (int b = 0; b < 4; ++b)
                v |= static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b8(rp, al + 4u * d + b, 0, 0)) << (8 * b);
            cw[l][d] = v;
        }
    };

#pragma unroll
    for (int l = 0; l < kLayers; ++l) {
        const std::uint32_t row = sh.rows[(wave * kLayers + l) * 8 + grp];
        cur[l] = end[l] = 0;
        int q = 0;
        roff[l] = 0.0f;
        if (row != kNoRow && fits) {
            const int b = a.row_ptr[row];
            // the code of entry e (relative to the block) starts at bit q + e * kBits
            q = (a.packed_row_ptr[row] - pk_al) * 8 - (b - wg_begin) * kBits;
            cur[l] = (a.row_start != nullptr ? a.row_start[row] : b) - wg_begin;
            end[l] = a.row_ptr[row + 1] - wg_begin;
            if constexpr (kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
                roff[l] = a.row_offsets != nullptr ? a.row_offsets[row] : 0.0f;
        }
        if (a.acc_init != nullptr && row != kNoRow) {
            head_init8(a, row, j, acc[l]);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[l][k] = 0.0f;
        }
        if (j == 0) sh.qbits[wave][l][grp] = q;
        load_window(l, q);
    }

    const char *wbase = reinterpret_cast<const char *>(sh.w) + j * 16;
    const char *mbase = reinterpret_cast<const char *>(sh.meta);
    uint4 *sp = &sh.u.stage[wave][grp][0];

    const int cols = static_cast<int>(a.cols);
    const int parts = (cols + kPartGenes - 1) / kPartGenes;
    for (int part = static_cast<int>(a.first_part); part < parts; ++part) {
        const int lo = part * kPartGenes;
        const int hi = lo + kPartGenes < cols ? lo + kPartGenes : cols;
        const std::uint32_t span = static_cast<std::uint32_t>(hi - lo);
        const std::uint32_t uhi = static_cast<std::uint32_t>(hi);
        __syncthreads();  // every wave is done reading part - 1
        load_part<kPolicy, kWaves>(sh, a, lo, hi, wave, lane, tid);  // also completes the window loads
        __syncthreads();
#pragma unroll
        for (int l = 0; l < kLayers; ++l) {
            for (;;) {
                if (tail) fix_tail(l);
                // the run: window entries with column < hi, entries past the row end excluded
                const int nv = end[l] - cur[l] - 8 * j;
                int n = 0;
                if (__builtin_amdgcn_ballot_w64(nv < 8) == 0u) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) n += colw[l][k] < uhi ? 1 : 0;
                } else {
#pragma unroll
                    for (int k = 0; k < 8; ++k) n += k < nv && colw[l][k] < uhi ? 1 : 0;
                }
                const int run = group_sum8i(n);
                const int rmax = wave_max_groups(run);
                const int ql = sh.qbits[wave][l][grp];
                const std::uint32_t bp = static_cast<std::uint32_t>(ql) + static_cast<std::uint32_t>(cur[l] + 8 * j) * kBits;
                const std::uint32_t c0 = __builtin_amdgcn_alignbit(cw[l][1], cw[l][0], bp & 31u);
                std::uint32_t c1 = 0u;
                if constexpr (kCodeDw == 3) c1 = __builtin_amdgcn_alignbit(cw[l][2], cw[l][1], bp & 31u);
                // The next window starts at the new cursor, known now. Its code dwords are
                // reloaded at once (this pass's codes are extracted above), its column slots
                // 0-3 once fill 1 has decoded them and slots 4-7 once fill 3 has: in a pass
                // that continues, the loads complete behind the remaining fills.
                const int next = cur[l] + run;
                const std::uint32_t e1 = static_cast<std::uint32_t>(next + 8 * j);
                load_codes(l, e1, ql);
                int okc = 0;
#pragma unroll
                for (int f = 0; f < 4; ++f) {
                    const bool live = 2 * f < rmax;
                    if (live) {
                        std::uint32_t st[4];
#pragma unroll
                        for (int r = 0; r < 2; ++r) {
                            const int k = 2 * f + r;
                            const std::uint32_t gk = colw[l][k] - static_cast<std::uint32_t>(lo);
                            // sorted columns (vouched for): a run entry lies in the part; the
                            // clamp only keeps a broken promise inside LDS
                            const bool ok = 8 * j + k < run && (kSorted || gk < span);
                            if constexpr (!kSorted) okc += ok ? 1 : 0;
                            const std::uint32_t gg = ok ? (kSorted ? min(gk, static_cast<std::uint32_t>(kPadGene)) : gk)
                                                        : static_cast<std::uint32_t>(kPadGene);
                            const float2 md = *reinterpret_cast<const float2 *>(mbase + gg * 8u);
                            std::uint32_t code;
                            if constexpr (kBits == 8) code = ((k < 4 ? c0 : c1) >> (8 * (k & 3))) & 0xffu;
                            else code = (c0 >> (k * kBits)) & kMask;
                            // pads read the (0, 0) metadata of the zero row: x = 0 without a branch
                            const float off = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET ? (ok ? roff[l] : 0.0f) : md.y;
                            const float x = __builtin_fmaf(static_cast<float>(code), md.x, off);
                            st[2 * r] = gg * 8u;
                            st[2 * r + 1] = __float_as_uint(x);
                        }
                        sp[j] = make_uint4(st[0], st[1], st[2], st[3]);
                    }
                    if (f == 1) load_cols(l, 0, e1);
                    if (f == 3) load_cols(l, 1, e1);
                    if (live) {
                        // pairs of stage slots, two pairs per iteration; an odd last slot alone
                        const int cnt = fill_count(rmax, f);
                        const int n2 = cnt >> 1;
                        int it = 0;
                        for (; it + 2 <= n2; it += 2) {
                            const uint4 ea = sp[it], eb = sp[it + 1];
                            const uint4 wa0 = *reinterpret_cast<const uint4 *>(wbase + (ea.x << 4));
                            const uint4 wa1 = *reinterpret_cast<const uint4 *>(wbase + (ea.z << 4));
                            const uint4 wb0 = *reinterpret_cast<const uint4 *>(wbase + (eb.x << 4));
                            const uint4 wb1 = *reinterpret_cast<const uint4 *>(wbase + (eb.z << 4));
                            fma8(acc[l], __uint_as_float(ea.y), wa0);
                            fma8(acc[l], __uint_as_float(ea.w), wa1);
                            fma8(acc[l], __uint_as_float(eb.y), wb0);
                            fma8(acc[l], __uint_as_float(eb.w), wb1);
                        }
                        if (it < n2) {
                            const uint4 e = sp[it];
                            const uint4 w0 = *reinterpret_cast<const uint4 *>(wbase + (e.x << 4));
                            const uint4 w1 = *reinterpret_cast<const uint4 *>(wbase + (e.z << 4));
                            fma8(acc[l], __uint_as_float(e.y), w0);
                            fma8(acc[l], __uint_as_float(e.w), w1);
                        }
                        if ((cnt & 1) != 0) {
                            const uint2 e = reinterpret_cast<const uint2 *>(sp)[cnt - 1];
                            fma8(acc[l], __uint_as_float(e.y), *reinterpret_cast<const uint4 *>(wbase + (e.x << 4)));
                        }
                    }
                }
                if constexpr (!kSorted) {
                    const int in_run = run - 8 * j < 0 ? 0 : (run - 8 * j > 8 ? 8 : run - 8 * j);
                    if (okc != in_run) end[l] = -1;  // broken: no further runs; recomputed at the end
                }
                cur[l] = next;
                const bool more = __builtin_amdgcn_ballot_w64(run == 64 && cur[l] < end[l]) != 0u;
                if (!more) break;
            }
        }
    }

#pragma unroll
    for (int l = 0; l < kLayers; ++l) {
        const std::uint32_t row = sh.rows[(wave * kLayers + l) * 8 + grp];
        const int bad = group_sum8i(cur[l] != end[l] || !fits ? 1 : 0);
        if (row != kNoRow && bad == 0) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                v[k] = a.ep.active ? epilogue_value(a.ep, acc[l][k], row, 8 * j + k) : acc[l][k];
            float4 *o = reinterpret_cast<float4 *>(a.out + static_cast<std::int64_t>(row) * a.out_ld + 8 * j);
            o[0] = make_float4(v[0], v[1], v[2], v[3]);
            o[1] = make_float4(v[4], v[5], v[6], v[7]);
        }
        // unfinished rows: recompute on the plain path (lane = column), one row at a time
        std::uint64_t todo = __builtin_amdgcn_ballot_w64(j == 0 && row != kNoRow && bad != 0);
        while (todo != 0u) {
            const int g = __builtin_ctzll(todo) >> 3;
            todo &= todo - 1u;
            const std::uint32_t r = sh.rows[(wave * kLayers + l) * 8 + g];
            const float v = row_fallback<kBits, kPolicy>(a, r, lane);
            a.out[static_cast<std::int64_t>(r) * a.out_ld + lane] = a.ep.active ? epilogue_value(a.ep, v, r, lane) : v;
        }
    }
}

// ---- the row-group walk over a prepared tail stream ------------------------------------------
//
// Same rows per lane group, registers, part copies and step loop as qcsr_spmm_groups, but the
// entries come prepared (qcsr_stream.hip): for each (block, part, wave, layer) the layer's
// runs are stored as fills of 16 steps x 8 lane groups in the order the stage holds them,
// and the fill index gives their position and the last fill's step count. So a pass loads
// one dword (two entries) per lane per fill, decodes it into the stage and steps; there is
// no window, run count or reload, and no per-row fallback (the builder rejects what the
// walk could not finish). The builder orders each group's run by gene parity, even-first in
// even groups and odd-first in odd groups: a weight row of gene g covers the LDS bank half
// g & 1, and groups 2i and 2i+1 read in the same LDS cycle, so their reads fall in
// different halves until one of them runs out of its preferred parity.

struct StreamShared {
    uint4 stage[kStreamWaves][8][9];  // per wave and lane group: 16 (gene * 8, value) pairs (+16 B pad)
    float2 meta[kPartGenes + 2];      // (scale, offset) per gene of the part; the two pads (0, 0)
    uint4 w[(kPartGenes + 2) * 8];    // fp16 weight rows of the part; the two pad rows are zeros
};

static_assert(kPadGene == static_cast<int>(kStreamPad) && kPadGene + 1 == static_cast<int>(kStreamPadOdd)
              && kPartGenes == kStreamPartGenes, "the stream builder and the part walk must agree on parts and pads");
// One workgroup per CU holds the whole part: gfx950's 160 KB of LDS per workgroup.
static_assert(sizeof(StreamShared) <= 160u * 1024u, "the tail walk's LDS exceeds gfx950's 160 KB");
static_assert(sizeof(GroupsShared<16, 4>) <= 160u * 1024u, "the row-group walk's LDS exceeds gfx950's 160 KB");

// Entries of one lane for one fill: group g's stage slots 2j, 2j + 1.
template<bool kWide>
struct FillWord {
    std::uint32_t w[kWide ? 2 : 1];
};

template<bool kWide>
__device__ __forceinline__ FillWord<kWide> load_fill(rsrc_t r, std::uint32_t offset) {
    FillWord<kWide> q;
    if constexpr (kWide) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, offset, 0, 0);
        q.w[0] = v[0];
        q.w[1] = v[1];
    } else {
        q.w[0] = static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, 0));
    }
    return q;
}

template<int kBits, int kPolicy>
__global__ __launch_bounds__(kStreamWaves * kWave) void qcsr_spmm_stream(QcsrArgs a) {
    constexpr int kWaves = kStreamWaves, kLayers = kStreamLayers;
    constexpr bool kWide = kBits == 8;
    constexpr std::uint32_t kFillBytes = kWide ? 512u : 256u;
    __shared__ StreamShared sh;
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int grp = lane >> 3;
    const int j = lane & 7;
    const std::uint32_t block = blockIdx.x;

    if (tid < 16) sh.w[kPadGene * 8 + tid] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 16 || tid == 17) sh.meta[kPadGene + tid - 16] = make_float2(0.0f, 0.0f);

    const int parts = static_cast<int>(a.stream_parts);
    const std::uint32_t *ix = a.fill_index + static_cast<std::uint64_t>(block) * parts * kStreamSlots;
    const std::uint32_t blk_first = __builtin_amdgcn_readfirstlane(ix[0]) & kFillMask;
    const std::uint32_t blk_end =
        __builtin_amdgcn_readfirstlane(ix[static_cast<std::uint64_t>(parts) * kStreamSlots]) & kFillMask;
    // This wave's index entries, (part, layer) order; entry parts * kLayers is the first fill
    // after the wave's (the next wave's, or the next block's, first).
    const std::uint32_t *wx = ix + static_cast<std::uint64_t>(wave) * parts * kLayers;
    const rsrc_t rx = make_rsrc(wx, static_cast<std::uint32_t>(parts * kLayers + 1) * 4u);
    const std::uint32_t ix_lane = static_cast<std::uint32_t>(lane <= kLayers ? lane : kLayers) * 4u;
    // the block's fills, addressed by 32-bit offsets (the builder bounds a block's bytes)
    const rsrc_t re = make_rsrc(static_cast<const char *>(a.stream_entries) + static_cast<std::uint64_t>(blk_first) * kFillBytes,
                                (blk_end - blk_first) * kFillBytes);
    const std::uint32_t lane_off = static_cast<std::uint32_t>(grp * 16 + 2 * j) * (kWide ? 4u : 2u);

    float acc[kLayers][8];
    float roff[kLayers];
    std::uint32_t rows[kLayers];
#pragma unroll
    for (int l = 0; l < kLayers; ++l) {
        const std::uint32_t row = a.slot_rows[static_cast<std::uint64_t>(block) * kStreamRows + (wave * kLayers + l) * 8 + grp];
        rows[l] = row;
        roff[l] = 0.0f;
        if constexpr (kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
            roff[l] = row != kNoRow && a.row_offsets != nullptr ? a.row_offsets[row] : 0.0f;
        if (a.acc_init != nullptr && row != kNoRow) {
            head_init8(a, row, j, acc[l]);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[l][k] = 0.0f;
        }
    }

    const char *wbase = reinterpret_cast<const char *>(sh.w) + j * 16;
    const char *mbase = reinterpret_cast<const char *>(sh.meta);
    uint4 *sp = &sh.stage[wave][grp][0];
    const int cols = static_cast<int>(a.cols);

    // The wave's fills are contiguous through all its parts, so the fill words load three
    // fills ahead without a restart at a part boundary. Each part's index entries (one per
    // lane, lanes 0 .. kLayers) load one part ahead, under the part before.
    std::uint32_t nb = __builtin_amdgcn_raw_buffer_load_b32(rx, ix_lane, 0, 0);
    std::uint32_t f = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(nb, 0)) & kFillMask;
    FillWord<kWide> q0 = load_fill<kWide>(re, (f - blk_first) * kFillBytes + lane_off);
    FillWord<kWide> q1 = load_fill<kWide>(re, (f + 1u - blk_first) * kFillBytes + lane_off);
    FillWord<kWide> q2 = load_fill<kWide>(re, (f + 2u - blk_first) * kFillBytes + lane_off);
    for (int p = 0; p < parts; ++p) {
        const int lo = (static_cast<int>(a.first_part) + p) * kPartGenes;
        const int hi = lo + kPartGenes < cols ? lo + kPartGenes : cols;
        __syncthreads();  // every wave is done reading part p - 1
        load_part<kPolicy, kWaves, StreamShared, false>(sh, a, lo, hi, wave, lane, tid);
        std::uint32_t b[kLayers + 1];
#pragma unroll
        for (int k = 0; k <= kLayers; ++k) b[k] = __builtin_amdgcn_readlane(nb, k);
        // the next part's entries (past the wave's last part: the entry after it, or zeros)
        nb = __builtin_amdgcn_raw_buffer_load_b32(rx, static_cast<std::uint32_t>((p + 1) * kLayers) * 4u + ix_lane, 0, 0);
        __builtin_amdgcn_s_waitcnt(0x0f71);  // vmcnt(1): the part copy and older loads; not the entries above
        __syncthreads();
#pragma unroll
        for (int l = 0; l < kLayers; ++l) {
            const std::uint32_t e_l = b[l + 1] & kFillMask;
            const int last = static_cast<int>(b[l] >> 28) + 1;
            for (; f < e_l; ++f) {
                const FillWord<kWide> cur = q0;
                q0 = q1;
                q1 = q2;
                q2 = load_fill<kWide>(re, (f + 3u - blk_first) * kFillBytes + lane_off);  // past the block: zeros, never used
                std::uint32_t st[4];
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    std::uint32_t g, code;
                    if constexpr (kWide) {
                        g = cur.w[r] & 0xffffu;
                        code = cur.w[r] >> 16;
                    } else {
                        const std::uint32_t e = r == 0 ? (cur.w[0] & 0xffffu) : (cur.w[0] >> 16);
                        g = e & 0x7ffu;
                        code = e >> 11;
                    }
                    g = min(g, static_cast<std::uint32_t>(kPadGene + 1));  // keeps a damaged stream inside LDS
                    const float2 md = *reinterpret_cast<const float2 *>(mbase + g * 8u);
                    const float off = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET
                        ? (g < static_cast<std::uint32_t>(kPadGene) ? roff[l] : 0.0f) : md.y;
                    st[2 * r] = g * 8u;
                    st[2 * r + 1] = __float_as_uint(__builtin_fmaf(static_cast<float>(code), md.x, off));
                }
                sp[j] = make_uint4(st[0], st[1], st[2], st[3]);
                // Steps in blocks of 4 stage slots; slots past a group's run hold pads (zero
                // row, value 0), so a block may run past `cnt`. A full fill is straight-line
                // code, which lets the weight reads of later blocks issue under earlier FMAs.
                // Keep the steps predicated in this one form: a separate unpredicated branch
                // for the fills before a layer's last was miscompiled by the ROCm 7.2 clang
                // (the decode's temporaries were allocated to registers holding live
                // accumulators, which the first step then read), giving wrong sums.
                auto step4 = [&](int q) {
                    const uint4 ea = sp[2 * q], eb = sp[2 * q + 1];
                    const uint4 wa0 = *reinterpret_cast<const uint4 *>(wbase + (ea.x << 4));
                    const uint4 wa1 = *reinterpret_cast<const uint4 *>(wbase + (ea.z << 4));
                    const uint4 wb0 = *reinterpret_cast<const uint4 *>(wbase + (eb.x << 4));
                    const uint4 wb1 = *reinterpret_cast<const uint4 *>(wbase + (eb.z << 4));
                    fma8(acc[l], __uint_as_float(ea.y), wa0);
                    fma8(acc[l], __uint_as_float(ea.w), wa1);
                    fma8(acc[l], __uint_as_float(eb.y), wb0);
                    fma8(acc[l], __uint_as_float(eb.w), wb1);
                };
                const int cnt = f + 1u < e_l ? 16 : last;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (4 * q < cnt) step4(q);
            }
        }
    }

#pragma unroll
    for (int l = 0; l < kLayers; ++l) {
        const std::uint32_t row = rows[l];
        if (row == kNoRow) continue;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = a.ep.active ? epilogue_value(a.ep, acc[l][k], row, 8 * j + k) : acc[l][k];
        float4 *o = reinterpret_cast<float4 *>(a.out + static_cast<std::int64_t>(row) * a.out_ld + 8 * j);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// ---- backward values in the row-group form -------------------------------------------------
//
// grad_values[i] = <G[row_i, :], W[col_i, :]> (64 columns) with the forward's row-group walk:
// lane group g owns one row of each layer and lane j holds G[row, 8j..8j+7] in registers;
// each pass counts the run, stages the run's weight-row offsets (pads: the zero row) in the
// forward's four fills, and per stage slot every lane multiplies its 8 columns with 16 B of
// the weight row; the 8 lanes' partial dots are summed (DPP) and lane j keeps the result
// of window entry 8j + k in register k, so each lane stores the 8 consecutive results of
// its own window slots (two 16-byte stores when the whole slot range is in the run).

struct BwdPartsArgs {
    const std::int32_t *row_ptr;
    const std::int32_t *col_idx;
    const float *grad_out;
    std::int64_t grad_out_ld;
    const std::uint16_t *rhs;  // fp16 [cols x 64]
    std::int64_t rhs_ld;
    float *grad_values;
    std::uint32_t rows;
    std::uint32_t cols;
};

// Sum over the 8 lanes of each lane group (quad xor 1, xor 2, then the half-row mirror).
__device__ __forceinline__ float group_sum8(float d) {
    d += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(d), 0xB1, 0xf, 0xf, false));
    d += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(d), 0x4E, 0xf, 0xf, false));
    d += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(d), 0x141, 0xf, 0xf, false));
    return d;
}

template<int kWaves, int kLayers>
struct BwdGroupsShared {
    static constexpr int kRows = kWaves * kLayers * 8;
    union {
        std::uint32_t stage[kWaves][8][20];  // per wave and lane group: 16 weight-row offsets (+16 B pad)
        GroupPrologue<kWaves, kLayers> pro;
    } u;
    uint4 w[(kPartGenes + 1) * 8];           // fp16 weight rows of the part; row kPadGene is zeros
    std::uint32_t rows[kRows];
};

__device__ __forceinline__ float dot8x2(const float (&g)[8], uint4 w) {
    float d0 = 0.0f, d1 = 0.0f;
    d0 = __builtin_fmaf(g[0], h2f(static_cast<std::uint16_t>(w.x & 0xffffu)), d0);
    d1 = __builtin_fmaf(g[1], h2f(static_cast<std::uint16_t>(w.x >> 16)), d1);
    d0 = __builtin_fmaf(g[2], h2f(static_cast<std::uint16_t>(w.y & 0xffffu)), d0);
    d1 = __builtin_fmaf(g[3], h2f(static_cast<std::uint16_t>(w.y >> 16)), d1);
    d0 = __builtin_fmaf(g[4], h2f(static_cast<std::uint16_t>(w.z & 0xffffu)), d0);
    d1 = __builtin_fmaf(g[5], h2f(static_cast<std::uint16_t>(w.z >> 16)), d1);
    d0 = __builtin_fmaf(g[6], h2f(static_cast<std::uint16_t>(w.w & 0xffffu)), d0);
    d1 = __builtin_fmaf(g[7], h2f(static_cast<std::uint16_t>(w.w >> 16)), d1);
    return d0 + d1;
}

template<int kWaves, int kLayers, bool kSorted>
__global__ __launch_bounds__(kWaves * kWave) void qcsr_bwd_values_groups(BwdPartsArgs a) {
    using Shared = BwdGroupsShared<kWaves, kLayers>;
    constexpr int kRows = Shared::kRows;
    __shared__ Shared sh;
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int grp = lane >> 3;
    const int j = lane & 7;
    const std::uint32_t first = blockIdx.x * static_cast<std::uint32_t>(kRows);
    const std::uint32_t last = first + kRows < a.rows ? first + kRows : a.rows;

    if (tid < 8) sh.w[kPadGene * 8 + tid] = make_uint4(0u, 0u, 0u, 0u);
    assign_groups<kWaves, kLayers>(sh.u.pro, sh.rows, a.row_ptr, a.rows, first, tid);

    const int wg_begin = __builtin_amdgcn_readfirstlane(a.row_ptr[first]);
    const int wg_end = __builtin_amdgcn_readfirstlane(a.row_ptr[last]);
    const bool fits = wg_end - wg_begin < (1 << 27);
    // Windows read up to 63 entries past the block (where the array goes on); the tail
    // block reloads windows that reach past the array end a dword at a time.
    const int nnz_all = __builtin_amdgcn_readfirstlane(a.row_ptr[a.rows]);
    const int col_n = nnz_all - wg_end < 72 ? nnz_all - wg_begin : wg_end - wg_begin + 72;
    const bool tail = nnz_all - wg_end < 72;
    const std::uint32_t col_lim = fits ? static_cast<std::uint32_t>(col_n) * 4u : 0u;
    const rsrc_t rc = make_rsrc(a.col_idx + wg_begin, col_lim);
    const rsrc_t ro = make_rsrc(a.grad_values + wg_begin, fits ? static_cast<std::uint32_t>(wg_end - wg_begin) * 4u : 0u);

    float g[kLayers][8];
    std::uint32_t colw[kLayers][8];
    int cur[kLayers], end[kLayers];

    auto load_cols = [&](int l, int h, std::uint32_t e0) {
        const auto c = __builtin_amdgcn_raw_buffer_load_b128(rc, e0 * 4u + 16u * h, 0, 0);
        colw[l][4 * h] = c[0]; colw[l][4 * h + 1] = c[1]; colw[l][4 * h + 2] = c[2]; colw[l][4 * h + 3] = c[3];
    };
    auto fix_tail = [&](int l) {
        const std::uint32_t e0 = static_cast<std::uint32_t>(cur[l] + 8 * j);
        if (__builtin_amdgcn_ballot_w64(e0 * 4u + 32u > col_lim) == 0u) return;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            colw[l][k] = static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rc, (e0 + k) * 4u, 0, 0));
    };

#pragma unroll
    for (int l = 0; l < kLayers; ++l) {
        const std::uint32_t row = sh.rows[(wave * kLayers + l) * 8 + grp];
        cur[l] = end[l] = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) g[l][k] = 0.0f;
        if (row != kNoRow && fits) {
            cur[l] = a.row_ptr[row] - wg_begin;
            end[l] = a.row_ptr[row + 1] - wg_begin;
            const float4 *gp = reinterpret_cast<const float4 *>(a.grad_out + static_cast<std::int64_t>(row) * a.grad_out_ld + j * 8);
            const float4 g0 = gp[0], g1 = gp[1];
            g[l][0] = g0.x; g[l][1] = g0.y; g[l][2] = g0.z; g[l][3] = g0.w;
            g[l][4] = g1.x; g[l][5] = g1.y; g[l][6] = g1.z; g[l][7] = g1.w;
        }
        const std::uint32_t e0 = static_cast<std::uint32_t>(cur[l] + 8 * j);
        load_cols(l, 0, e0);
        load_cols(l, 1, e0);
    }

    const char *wbase = reinterpret_cast<const char *>(sh.w) + j * 16;
    std::uint32_t *sp = &sh.u.stage[wave][grp][0];

    const int cols = static_cast<int>(a.cols);
    const int parts = (cols + kPartGenes - 1) / kPartGenes;
    for (int part = 0; part < parts; ++part) {
        const int lo = part * kPartGenes;
        const int hi = lo + kPartGenes < cols ? lo + kPartGenes : cols;
        const std::uint32_t span = static_cast<std::uint32_t>(hi - lo);
        const std::uint32_t uhi = static_cast<std::uint32_t>(hi);
        __syncthreads();  // every wave is done reading part - 1
        load_part_weights<kWaves>(sh.w, a.rhs, a.rhs_ld, lo, hi, wave, lane);
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the copy (and the window loads)
        __syncthreads();
#pragma unroll
        for (int l = 0; l < kLayers; ++l) {
            for (;;) {
                if (tail) fix_tail(l);
                const int nv = end[l] - cur[l] - 8 * j;
                int n = 0;
                if (__builtin_amdgcn_ballot_w64(nv < 8) == 0u) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) n += colw[l][k] < uhi ? 1 : 0;
                } else {
#pragma unroll
                    for (int k = 0; k < 8; ++k) n += k < nv && colw[l][k] < uhi ? 1 : 0;
                }
                const int run = group_sum8i(n);
                const int rmax = wave_max_groups(run);
                const int next = cur[l] + run;
                const std::uint32_t e1 = static_cast<std::uint32_t>(next + 8 * j);
                float res[8];
                int okc = 0;
#pragma unroll
                for (int f = 0; f < 4; ++f) {
                    const bool live = 2 * f < rmax;
                    if (live) {
                        std::uint32_t st[2];
#pragma unroll
                        for (int r = 0; r < 2; ++r) {
                            const int k = 2 * f + r;
                            const std::uint32_t gk = colw[l][k] - static_cast<std::uint32_t>(lo);
                            const bool ok = 8 * j + k < run && (kSorted || gk < span);
                            if constexpr (!kSorted) okc += ok ? 1 : 0;
                            st[r] = (ok ? (kSorted ? min(gk, static_cast<std::uint32_t>(kPadGene)) : gk)
                                        : static_cast<std::uint32_t>(kPadGene)) * 128u;
                        }
                        *reinterpret_cast<uint2 *>(sp + 2 * j) = make_uint2(st[0], st[1]);
                    }
                    if (f == 1) load_cols(l, 0, e1);
                    if (f == 3) load_cols(l, 1, e1);
                    if (live) {
                        // stage slot pair `it` holds window entries 8 it + 2f and 8 it + 2f + 1:
                        // lane it of the group keeps their results in res[2f], res[2f + 1]
                        const int n2 = (fill_count(rmax, f) + 1) >> 1;
                        res[2 * f] = res[2 * f + 1] = 0.0f;
                        int it = 0;
                        for (; it + 2 <= n2; it += 2) {
                            const uint4 e = reinterpret_cast<const uint4 *>(sp)[it >> 1];
                            const uint4 w0 = *reinterpret_cast<const uint4 *>(wbase + e.x);
                            const uint4 w1 = *reinterpret_cast<const uint4 *>(wbase + e.y);
                            const uint4 w2 = *reinterpret_cast<const uint4 *>(wbase + e.z);
                            const uint4 w3 = *reinterpret_cast<const uint4 *>(wbase + e.w);
                            const float d0 = group_sum8(dot8x2(g[l], w0));
                            const float d1 = group_sum8(dot8x2(g[l], w1));
                            const float d2 = group_sum8(dot8x2(g[l], w2));
                            const float d3 = group_sum8(dot8x2(g[l], w3));
                            if (j == it) {
                                res[2 * f] = d0;
                                res[2 * f + 1] = d1;
                            }
                            if (j == it + 1) {
                                res[2 * f] = d2;
                                res[2 * f + 1] = d3;
                            }
                        }
                        if (it < n2) {
                            const uint2 e = reinterpret_cast<const uint2 *>(sp)[it];
                            const uint4 w0 = *reinterpret_cast<const uint4 *>(wbase + e.x);
                            const uint4 w1 = *reinterpret_cast<const uint4 *>(wbase + e.y);
                            const float d0 = group_sum8(dot8x2(g[l], w0));
                            const float d1 = group_sum8(dot8x2(g[l], w1));
                            if (j == it) {
                                res[2 * f] = d0;
                                res[2 * f + 1] = d1;
                            }
                        }
                    }
                }
                // this lane's window slots in the run: entries cur + 8j .. cur + 8j + in_run - 1
                const int in_run = run - 8 * j < 0 ? 0 : (run - 8 * j > 8 ? 8 : run - 8 * j);
                const std::uint32_t o0 = static_cast<std::uint32_t>(cur[l] + 8 * j) * 4u;
                if (in_run == 8) {
                    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                    const u32x4 lo4 = {__float_as_uint(res[0]), __float_as_uint(res[1]), __float_as_uint(res[2]),
                                       __float_as_uint(res[3])};
                    const u32x4 hi4 = {__float_as_uint(res[4]), __float_as_uint(res[5]), __float_as_uint(res[6]),
                                       __float_as_uint(res[7])};
                    __builtin_amdgcn_raw_buffer_store_b128(lo4, ro, o0, 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b128(hi4, ro, o0 + 16u, 0, 0);
                } else {
#pragma unroll
                    for (int k = 0; k < 8; ++k)
                        if (k < in_run) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(res[k]), ro, o0 + 4u * k, 0, 0);
                }
                if constexpr (!kSorted)
                    if (okc != in_run) end[l] = -1;  // broken: no further runs; recomputed at the end
                cur[l] = next;
                if (__builtin_amdgcn_ballot_w64(run == 64 && cur[l] < end[l]) == 0u) break;
            }
        }
    }

    // rows the walk could not finish: the whole row again on a plain path (lane = column;
    // columns outside [0, cols) give 0), after this wave's stores above have completed
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int l = 0; l < kLayers; ++l) {
        const std::uint32_t row = sh.rows[(wave * kLayers + l) * 8 + grp];
        const int bad = group_sum8i(cur[l] != end[l] || !fits ? 1 : 0);
        std::uint64_t todo = __builtin_amdgcn_ballot_w64(j == 0 && row != kNoRow && bad != 0);
        while (todo != 0u) {
            const int gsel = __builtin_ctzll(todo) >> 3;
            todo &= todo - 1u;
            const std::uint32_t r = sh.rows[(wave * kLayers + l) * 8 + gsel];
            const float gl = a.grad_out[static_cast<std::int64_t>(r) * a.grad_out_ld + lane];
            for (int i = a.row_ptr[r]; i < a.row_ptr[r + 1]; ++i) {
                const std::uint32_t col = static_cast<std::uint32_t>(a.col_idx[i]);
                float d = col < a.cols ? gl * h2f(a.rhs[static_cast<std::int64_t>(col) * a.rhs_ld + lane]) : 0.0f;
                d = xor_reduce<0, 5>(d);
                if (lane == 0) a.grad_values[i] = d;
            }
        }
    }
}

template<int kBits, int kPolicy>
int launch_bits_groups(const QcsrArgs &a, hipStream_t stream) {
    constexpr int kWaves = 16, kLayers = 4;
    const dim3 grid(round_block_count(a.rows, kWaves * kLayers * 8, blocks_per_round(), true)), block(kWaves * kWave);
    if ((a.flags & CX_QCSR_COLUMNS_SORTED) != 0u)
        hipLaunchKernelGGL((qcsr_spmm_groups<kBits, kPolicy, kWaves, kLayers, true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((qcsr_spmm_groups<kBits, kPolicy, kWaves, kLayers, false>), grid, block, 0, stream, a);
    return check_launch("qcsr_spmm_groups");
}

template<int kPolicy>
int launch_policy_parts(const QcsrArgs &a, std::uint32_t bits, hipStream_t stream) {
    switch (bits) {
    case 1: return launch_bits_groups<1, kPolicy>(a, stream);
    case 2: return launch_bits_groups<2, kPolicy>(a, stream);
    case 4: return launch_bits_groups<4, kPolicy>(a, stream);
    default: return launch_bits_groups<8, kPolicy>(a, stream);
    }
}

} // namespace

bool qcsr_parts_applicable(const QcsrArgs &a, std::uint32_t bits, std::uint32_t rhs_dtype,
                           std::int64_t out_cols, bool aligned) {
    return bits != 0u && rhs_dtype == CELLERATOR_DTYPE_F16 && out_cols > 0 && out_cols % 64 == 0
        && out_cols <= 256 && aligned && a.cols <= static_cast<std::uint32_t>(INT32_MAX) && a.rows > 0u && a.cols > 0u
        && a.rhs_ld <= (INT32_MAX / 2) / kPartGenes;
}

// N = 64 c columns: one launch per 64-column block of the weights and the output (and of
// the epilogue's bias and initial values).
bool bwd_values_parts_applicable(std::uint32_t rows, std::uint32_t cols, std::uint32_t rhs_dtype,
                                 std::int64_t out_cols, bool aligned, std::int64_t rhs_ld) {
    return rhs_dtype == CELLERATOR_DTYPE_F16 && out_cols == 64 && aligned && rows > 0u && cols > 0u
        && cols <= static_cast<std::uint32_t>(INT32_MAX) && rhs_ld <= (INT32_MAX / 2) / kPartGenes;
}

int launch_bwd_values_parts(const std::int32_t *row_ptr, const std::int32_t *col_idx, const float *grad_out,
                            std::int64_t grad_out_ld, const void *rhs, std::int64_t rhs_ld,
                            float *grad_values, std::uint32_t rows, std::uint32_t cols, bool sorted,
                            hipStream_t stream) {
    constexpr int kWaves = 16, kLayers = 4;
    const BwdPartsArgs a{row_ptr, col_idx, grad_out, grad_out_ld, static_cast<const std::uint16_t *>(rhs), rhs_ld,
                         grad_values, rows, cols};
    const unsigned rows_per_block = kWaves * kLayers * 8;
    const dim3 grid((rows + rows_per_block - 1) / rows_per_block), block(kWaves * kWave);
    if (sorted)
        hipLaunchKernelGGL((qcsr_bwd_values_groups<kWaves, kLayers, true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((qcsr_bwd_values_groups<kWaves, kLayers, false>), grid, block, 0, stream, a);
    return check_launch("qcsr_bwd_values_groups");
}

int launch_qcsr_stream(const QcsrArgs &a, std::uint32_t bits, std::uint32_t policy, hipStream_t stream) {
    const dim3 grid(a.stream_blocks), block(kStreamWaves * kWave);
#define CX_STREAM(B, P) hipLaunchKernelGGL((qcsr_spmm_stream<B, P>), grid, block, 0, stream, a)
#define CX_STREAM_POLICY(B)                                                                         \
    do {                                                                                            \
        if (policy == CX_DECODE_PER_GENE_AFFINE_PAIRS) CX_STREAM(B, CX_DECODE_PER_GENE_AFFINE_PAIRS);   \
        else if (policy == CX_DECODE_PER_GENE_AFFINE) CX_STREAM(B, CX_DECODE_PER_GENE_AFFINE);          \
        else CX_STREAM(B, CX_DECODE_COLUMN_SCALE_ROW_OFFSET);                                           \
    } while (0)
    switch (bits) {
    case 1: CX_STREAM_POLICY(1); break;
    case 2: CX_STREAM_POLICY(2); break;
    case 4: CX_STREAM_POLICY(4); break;
    default: CX_STREAM_POLICY(8); break;
    }
#undef CX_STREAM_POLICY
#undef CX_STREAM
    return check_launch("qcsr_spmm_stream");
}

int launch_qcsr_parts(const QcsrArgs &a, std::uint32_t bits, std::uint32_t policy, std::int64_t out_cols,
                      hipStream_t stream) {
    for (std::int64_t c0 = 0; c0 < out_cols; c0 += 64) {
        QcsrArgs b = a;
        b.rhs = static_cast<const std::uint16_t *>(a.rhs) + c0;
        b.out = a.out + c0;
        if (b.ep.bias != nullptr) b.ep.bias += c0;
        if (b.ep.initial != nullptr) b.ep.initial += c0;
        int rc;
        if (policy == CX_DECODE_PER_GENE_AFFINE_PAIRS)
            rc = launch_policy_parts<CX_DECODE_PER_GENE_AFFINE_PAIRS>(b, bits, stream);
        else if (policy == CX_DECODE_PER_GENE_AFFINE)
            rc = launch_policy_parts<CX_DECODE_PER_GENE_AFFINE>(b, bits, stream);
        else
            rc = launch_policy_parts<CX_DECODE_COLUMN_SCALE_ROW_OFFSET>(b, bits, stream);
        if (rc != CX_STATUS_SUCCESS) return rc;
    }
    return CX_STATUS_SUCCESS;
}

} // namespace cx
