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
// kernel). Backward values (qcsr_bwd_values_parts): all 8 lane groups of a wave work on one
// row at a time, each group on a different entry, with the row's gradient in registers.
#include "qcsr_common.hpp"

namespace cx {
namespace {

constexpr int kPartGenes = 1024;                 // 128 KB of fp16 weight rows per part
constexpr std::uint32_t kNoGene = 0xffffffffu;   // never inside a part
constexpr std::uint32_t kNoRow = 0xffffffffu;
constexpr int kRefill = 48;                      // refill a row's window below this many

using rsrc_t = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, std::uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

using lds_ptr = __attribute__((address_space(3))) void *;

// The weight rows and metadata of genes [lo, hi) into LDS. The weight rows go straight from
// memory to LDS (buffer loads with the lds flag: wave instruction k of wave w fills 1 KB,
// 8 rows, at no register cost); loads past the part's last row return zeros. Interleaved
// (scale, offset) pairs go the same way; the other decode policies build their pairs in
// registers.
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
template<int kPolicy, int kWaves, typename Shared>
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
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the LDS writes of the loads above
}

// Snake assignment of a block's rows to waves: rank the rows by length (descending, ties
// by index) and deal rank r to slot r / kWaves of wave (r / kWaves even ? r % kWaves
// : kWaves - 1 - r % kWaves), so every wave carries about the same number of nonzeros.
template<int kWaves, int kRw>
__device__ __forceinline__ void assign_rows(int *len, std::uint32_t *rows_out, const std::int32_t *row_ptr,
                                            std::uint32_t rows, std::uint32_t first, int tid) {
    constexpr int kBlockRows = kWaves * kRw;
    if (tid < kBlockRows) {
        const std::uint32_t row = first + static_cast<std::uint32_t>(tid);
        len[tid] = row < rows ? row_ptr[row + 1] - row_ptr[row] : -1;
    }
    __syncthreads();
    if (tid < kBlockRows) {
        const int my = len[tid];
        int rank = 0;
#pragma unroll 4
        for (int u = 0; u < kBlockRows; ++u) {
            const int lu = len[u];
            rank += lu > my || (lu == my && u < tid) ? 1 : 0;
        }
        const int round = rank / kWaves, pos = rank % kWaves;
        const int w = (round & 1) != 0 ? kWaves - 1 - pos : pos;
        const std::uint32_t row = first + static_cast<std::uint32_t>(tid);
        rows_out[w * kRw + round] = row < rows ? row : kNoRow;
    }
    __syncthreads();
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
template<int kBits, int kPolicy>
__device__ float row_fallback(const QcsrArgs &a, std::uint32_t row, int lane) {
    const std::int64_t begin = a.row_ptr[row], end = a.row_ptr[row + 1];
    const std::uint8_t *pbase = a.packed + a.packed_row_ptr[row];
    const float row_offset = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET && a.row_offsets != nullptr
        ? a.row_offsets[row] : 0.0f;
    const std::uint16_t *rhs = static_cast<const std::uint16_t *>(a.rhs);
    float acc = 0.0f;
    for (std::int64_t i = begin; i < end; ++i) {
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

template<int kWaves, int kLayers>
struct GroupsShared {
    static constexpr int kRows = kWaves * kLayers * 8;
    union {
        uint4 stage[kWaves][8][9];  // per wave and lane group: 16 (metadata byte offset, value) pairs (+16 B pad)
        int len[kRows];             // prologue: row lengths
    } u;
    float2 meta[kPartGenes + 2];    // (scale, offset) per gene of the part; [kPadGene] = (0, 0)
    uint4 w[(kPartGenes + 1) * 8];  // fp16 weight rows of the part; row kPadGene is zeros
    std::uint32_t rows[kRows];      // row of (wave, layer, group)
    int qbits[kWaves][kLayers][8];  // code bit offset q of (wave, layer, group): kept here, not in registers
};

// Rank the block's rows by length (descending, ties by index); ranks 8s .. 8s + 7 form row
// set s (similar lengths, so the 8 groups of a layer finish their runs together), and the
// sets are dealt to the waves in snake order (set s -> layer s / kWaves), so every wave
// carries about the same number of nonzeros.
template<int kWaves, int kLayers>
__device__ __forceinline__ void assign_groups(int *len, std::uint32_t *rows_out, const std::int32_t *row_ptr,
                                              std::uint32_t rows, std::uint32_t first, int tid) {
    constexpr int kRows = kWaves * kLayers * 8;
    const std::uint32_t row = first + static_cast<std::uint32_t>(tid);
    if (tid < kRows) len[tid] = row < rows ? row_ptr[row + 1] - row_ptr[row] : -1;
    __syncthreads();
    if (tid < kRows) {
        const int my = len[tid];
        int rank = 0;
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
        const int set = rank / 8, g = rank % 8;
        const int round = set / kWaves, pos = set % kWaves;
        const int w = (round & 1) != 0 ? kWaves - 1 - pos : pos;
        rows_out[(w * kLayers + round) * 8 + g] = row < rows ? row : kNoRow;
    }
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

template<int kBits, int kPolicy, int kWaves, int kLayers>
__global__ __launch_bounds__(kWaves * kWave) void qcsr_spmm_groups(QcsrArgs a) {
    using Shared = GroupsShared<kWaves, kLayers>;
    constexpr int kRows = Shared::kRows;
    constexpr int kCodeDw = kBits == 8 ? 3 : 2;
    constexpr std::uint32_t kMask = (1u << kBits) - 1u;
    __shared__ Shared sh;
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int grp = lane >> 3;
    const int j = lane & 7;
    const std::uint32_t first = blockIdx.x * static_cast<std::uint32_t>(kRows);
    const std::uint32_t last = first + kRows < a.rows ? first + kRows : a.rows;

    if (tid < 8) sh.w[kPadGene * 8 + tid] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 8) sh.meta[kPadGene] = make_float2(0.0f, 0.0f);
    assign_groups<kWaves, kLayers>(sh.u.len, sh.rows, a.row_ptr, a.rows, first, tid);

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
            cur[l] = b - wg_begin;
            end[l] = a.row_ptr[row + 1] - wg_begin;
            q = (a.packed_row_ptr[row] - pk_al) * 8 - cur[l] * kBits;
            if constexpr (kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
                roff[l] = a.row_offsets != nullptr ? a.row_offsets[row] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[l][k] = 0.0f;
        if (j == 0) sh.qbits[wave][l][grp] = q;
        load_window(l, q);
    }

    const char *wbase = reinterpret_cast<const char *>(sh.w) + j * 16;
    const char *mbase = reinterpret_cast<const char *>(sh.meta);
    uint4 *sp = &sh.u.stage[wave][grp][0];

    const int cols = static_cast<int>(a.cols);
    const int parts = (cols + kPartGenes - 1) / kPartGenes;
    for (int part = 0; part < parts; ++part) {
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
                            const bool ok = 8 * j + k < run && gk < span;
                            okc += ok ? 1 : 0;
                            const std::uint32_t gg = ok ? gk : static_cast<std::uint32_t>(kPadGene);
                            const float2 md = *reinterpret_cast<const float2 *>(mbase + gg * 8u);
                            std::uint32_t code;
                            if constexpr (kBits == 8) code = ((k < 4 ? c0 : c1) >> (8 * (k & 3))) & 0xffu;
                            else code = (c0 >> (k * kBits)) & kMask;
                            const float off = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET ? roff[l] : md.y;
                            const float x = ok ? __builtin_fmaf(static_cast<float>(code), md.x, off) : 0.0f;
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
                const int in_run = run - 8 * j < 0 ? 0 : (run - 8 * j > 8 ? 8 : run - 8 * j);
                if (okc != in_run) end[l] = -1;  // broken: no further runs; recomputed at the end
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

// ---- backward values: grad_values[i] = <G[row_i, :], W[col_i, :]> over 64 columns --------
//
// The same part walk without decode (the gradient does not depend on the stored values):
// each wave keeps its rows' G (lane j: columns 8j..8j+7, fp32) in registers; lane group g
// takes staged entry s + g, lane j multiplies its 8 columns with 16 B of the LDS weight
// row, the group sums its 8 lanes (DPP), and the dots are staged and stored coalesced per
// visit.

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

template<int kWaves, int kRw>
struct BwdPartsShared {
    uint4 w[kPartGenes * 8];          // [gene][16-byte quarter-rows]: fp16 weights
    int stage[kWaves][2][kWave];      // per wave, two rows: LDS byte offset of the weight row
    float dots[kWaves][2][kWave];     // per wave, two rows: the staged entries' results
    int len[kWaves * kRw];
    std::uint32_t rows[kWaves * kRw];
};

__device__ __forceinline__ float dot8(const float (&g)[8], uint4 w) {
    const std::uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float d = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        d = __builtin_fmaf(g[2 * k], h2f(static_cast<std::uint16_t>(words[k] & 0xffffu)), d);
        d = __builtin_fmaf(g[2 * k + 1], h2f(static_cast<std::uint16_t>(words[k] >> 16)), d);
    }
    return d;
}

// Sum over the 8 lanes of each lane group (quad xor 1, xor 2, then the half-row mirror).
__device__ __forceinline__ float group_sum8(float d) {
    d += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(d), 0xB1, 0xf, 0xf, false));
    d += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(d), 0x4E, 0xf, 0xf, false));
    d += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(d), 0x141, 0xf, 0xf, false));
    return d;
}

template<int kWaves, int kRw>
__global__ __launch_bounds__(kWaves * kWave) void qcsr_bwd_values_parts(BwdPartsArgs a) {
    constexpr int kBlockRows = kWaves * kRw;
    static_assert(kBlockRows <= kWaves * kWave && kRw <= kWave && kRw % 2 == 0, "bad part-kernel shape");
    __shared__ BwdPartsShared<kWaves, kRw> sh;
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int grp = lane >> 3;
    const int j = lane & 7;
    const std::uint32_t first = blockIdx.x * static_cast<std::uint32_t>(kBlockRows);
    assign_rows<kWaves, kRw>(sh.len, sh.rows, a.row_ptr, a.rows, first, tid);
    const int nnz = __builtin_amdgcn_readfirstlane(a.row_ptr[a.rows]);

    int cur[kRw], end[kRw], base[kRw];
    float g[kRw][8];
    std::uint32_t win[kRw];
    auto load_cols = [&](int rw) {  // window: column indices of entries [base, base + 64)
        const std::uint32_t ub = static_cast<std::uint32_t>(base[rw]);
        const std::uint32_t n = static_cast<std::uint32_t>(nnz) - ub < kWave ? static_cast<std::uint32_t>(nnz) - ub : kWave;
        win[rw] = static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(
            make_rsrc(a.col_idx + ub, n * 4u), lane * 4, 0, 0));
    };
#pragma unroll
    for (int rw = 0; rw < kRw; ++rw) {
        const std::uint32_t row = __builtin_amdgcn_readfirstlane(sh.rows[wave * kRw + rw]);
        cur[rw] = end[rw] = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) g[rw][k] = 0.0f;
        if (row != kNoRow) {
            cur[rw] = __builtin_amdgcn_readfirstlane(a.row_ptr[row]);
            end[rw] = __builtin_amdgcn_readfirstlane(a.row_ptr[row + 1]);
            const float4 *gp = reinterpret_cast<const float4 *>(a.grad_out + static_cast<std::int64_t>(row) * a.grad_out_ld + j * 8);
            const float4 g0 = gp[0], g1 = gp[1];
            g[rw][0] = g0.x; g[rw][1] = g0.y; g[rw][2] = g0.z; g[rw][3] = g0.w;
            g[rw][4] = g1.x; g[rw][5] = g1.y; g[rw][6] = g1.z; g[rw][7] = g1.w;
        }
        base[rw] = cur[rw];
        win[rw] = kNoGene;
        if (cur[rw] < end[rw]) load_cols(rw);
    }
    const char *wbase = reinterpret_cast<const char *>(sh.w) + j * 16;

    auto segment = [&](int rw, int lo, std::uint32_t span, int &start, int &cnt, std::uint32_t &gl) {
        start = cur[rw] - base[rw];
        gl = win[rw] - static_cast<std::uint32_t>(lo);
        const std::uint64_t run = ~(__builtin_amdgcn_ballot_w64(gl < span) >> start);
        const int in_run = run == 0u ? kWave - start : __builtin_ctzll(run);
        cnt = in_run < end[rw] - cur[rw] ? in_run : end[rw] - cur[rw];
    };
    auto stage = [&](int slot, int start, int cnt, std::uint32_t gl) {
        if (static_cast<std::uint32_t>(lane - start) < static_cast<std::uint32_t>(cnt))
            sh.stage[wave][slot][lane] = static_cast<int>(gl) * 128;
    };
    // dots of staged entries [start, start + cnt) of slot `slot` into sh.dots
    auto step1 = [&](int rw, int slot, int s) {
        const int e = sh.stage[wave][slot][s + grp];
        const float d = group_sum8(dot8(g[rw], *reinterpret_cast<const uint4 *>(wbase + e)));
        if (j == 0) sh.dots[wave][slot][s + grp] = d;
    };
    auto dots = [&](int rw, int slot, int s, int stop) {
        for (; s + 8 <= stop; s += 8) step1(rw, slot, s);
        if (s + grp < stop) step1(rw, slot, s);
    };
    auto store = [&](int rw, int slot, int start, int cnt) {
        if (static_cast<std::uint32_t>(lane - start) < static_cast<std::uint32_t>(cnt))
            a.grad_values[static_cast<std::uint32_t>(base[rw] + lane)] = sh.dots[wave][slot][lane];
    };
    auto advance = [&](int rw, int stop, int cnt) -> bool {
        cur[rw] += cnt;
        if (stop < kWave || cur[rw] >= end[rw]) return false;
        base[rw] = cur[rw];
        load_cols(rw);
        return true;
    };
    auto visit_rest = [&](int rw, int lo, std::uint32_t span) {
        for (;;) {
            int start, cnt;
            std::uint32_t gl;
            segment(rw, lo, span, start, cnt, gl);
            if (cnt == 0) return;
            stage(0, start, cnt, gl);
            wave_sync();
            dots(rw, 0, start, start + cnt);
            wave_sync();
            store(rw, 0, start, cnt);
            if (!advance(rw, start + cnt, cnt)) return;
        }
    };
    auto refill = [&](int rw) {
        if (base[rw] + kWave < end[rw] && base[rw] + kWave - cur[rw] < kRefill) {
            base[rw] = cur[rw];
            load_cols(rw);
        }
    };

    const int cols = static_cast<int>(a.cols);
    const int parts = (cols + kPartGenes - 1) / kPartGenes;
    for (int part = 0; part < parts; ++part) {
        const int lo = part * kPartGenes;
        const int hi = lo + kPartGenes < cols ? lo + kPartGenes : cols;
        const std::uint32_t span = static_cast<std::uint32_t>(hi - lo);
        __syncthreads();  // every wave is done reading part - 1
        load_part_weights<kWaves>(sh.w, a.rhs, a.rhs_ld, lo, hi, wave, lane);
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the copy (and the window refills)
        __syncthreads();
#pragma unroll
        for (int ra = 0; ra < kRw; ra += 2) {
            const int rb = ra + 1;
            int sa = 0, ca = 0, sb = 0, cb = 0;
            std::uint32_t ga = 0u, gb = 0u;
            if (cur[ra] < end[ra]) segment(ra, lo, span, sa, ca, ga);
            if (cur[rb] < end[rb]) segment(rb, lo, span, sb, cb, gb);
            stage(0, sa, ca, ga);
            stage(1, sb, cb, gb);
            wave_sync();
            int s_a = sa, s_b = sb;
            const int stop_a = sa + ca, stop_b = sb + cb;
            for (; s_a + 8 <= stop_a && s_b + 8 <= stop_b; s_a += 8, s_b += 8) {
                step1(ra, 0, s_a);
                step1(rb, 1, s_b);
            }
            dots(ra, 0, s_a, stop_a);
            dots(rb, 1, s_b, stop_b);
            wave_sync();
            store(ra, 0, sa, ca);
            store(rb, 1, sb, cb);
            const bool more_a = ca > 0 && advance(ra, stop_a, ca);
            const bool more_b = cb > 0 && advance(rb, stop_b, cb);
            if (more_a) visit_rest(ra, lo, span);
            if (more_b) visit_rest(rb, lo, span);
            refill(ra);
            refill(rb);
        }
    }

    // rows the walk could not finish: the remaining entries on a plain path (lane = column;
    // columns outside [0, cols) give 0)
#pragma unroll
    for (int rw = 0; rw < kRw; ++rw) {
        if (cur[rw] >= end[rw]) continue;
        const std::uint32_t row = __builtin_amdgcn_readfirstlane(sh.rows[wave * kRw + rw]);
        const float gl = a.grad_out[static_cast<std::int64_t>(row) * a.grad_out_ld + lane];
        for (int i = cur[rw]; i < end[rw]; ++i) {
            const std::uint32_t col = static_cast<std::uint32_t>(a.col_idx[i]);
            float d = col < a.cols ? gl * h2f(a.rhs[static_cast<std::int64_t>(col) * a.rhs_ld + lane]) : 0.0f;
            d = xor_reduce<0, 5>(d);
            if (lane == 0) a.grad_values[i] = d;
        }
    }
}

template<int kBits, int kPolicy>
int launch_bits_groups(const QcsrArgs &a, hipStream_t stream) {
    constexpr int kWaves = 16, kLayers = 4;
    const unsigned rows_per_block = kWaves * kLayers * 8;
    const dim3 grid((a.rows + rows_per_block - 1) / rows_per_block), block(kWaves * kWave);
    hipLaunchKernelGGL((qcsr_spmm_groups<kBits, kPolicy, kWaves, kLayers>), grid, block, 0, stream, a);
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
                            float *grad_values, std::uint32_t rows, std::uint32_t cols, hipStream_t stream) {
    constexpr int kWaves = 16, kRw = 8;
    const BwdPartsArgs a{row_ptr, col_idx, grad_out, grad_out_ld, static_cast<const std::uint16_t *>(rhs), rhs_ld,
                         grad_values, rows, cols};
    const unsigned rows_per_block = kWaves * kRw;
    const dim3 grid((rows + rows_per_block - 1) / rows_per_block), block(kWaves * kWave);
    hipLaunchKernelGGL((qcsr_bwd_values_parts<kWaves, kRw>), grid, block, 0, stream, a);
    return check_launch("qcsr_bwd_values_parts");
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
