// qcsr_parts.hip -- quantized CSR SpMM with the weight panel streamed through LDS by gene
// part (fp16 weights, N a multiple of 64 in blocks of 64 columns, column-sorted rows).
//
// Same value semantics as qcsr_spmm.hip (decode fma(float(code), scale, offset), exact fp16
// widening, fp32 products and sums); only the summation order differs, and it is fixed.
//
// Why: gathering a 128-byte weight row per nonzero through the texture path, plus an
// 8-byte metadata gather per code, keeps the row-wave kernel far below HBM speed. LDS
// serves the same 16-byte-per-lane gathers at about twice the rate, and the per-gene
// metadata of a part sits beside its weight rows.
//
// Layout: one workgroup of kWaves waves per CU (LDS-bound) owns kWaves x kRw rows. A
// prologue ranks the block's rows by length and deals them to the waves in snake order,
// so every wave carries about the same number of nonzeros. The workgroup walks the genes in
// parts of kPartGenes:
//   * the part's fp16 weight rows (128 B each) and (scale, offset) pairs are copied into
//     LDS by buffer loads that write LDS directly;
//   * each wave then visits its rows, two at a time. Columns within a row are sorted, so
//     the row's entries in the part are the run starting at the row's cursor. The wave keeps
//     the next 64 entries of every row in two registers (column index, code byte), decodes
//     the run from the LDS metadata, stages (LDS offset of the weight row, value), and lets
//     lane group g = lane / 8 take entry s + g while lane j = lane % 8 reads 16 B of that
//     weight row and issues 8 v_fma_mix_f32 into the row's 8 partial sums;
//   * right after a pair's visits, each row window with fewer than kRefill entries left is
//     refilled; those loads complete behind the rest of the part.
// After the last part the 8 lane groups' partials of each row are reduce-scattered
// (permlane32 swap, permlane16 swap, DPP row rotate), leaving one column per lane.
// Rows whose cursor cannot advance (a column out of order across parts, or outside
// [0, cols)) are recomputed at the end on a plain per-row path that skips columns outside
// [0, cols); valid sorted input never takes it.
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

template<int kWaves, int kRw>
struct PartsShared {
    uint4 w[kPartGenes * 8];          // [gene][16-byte quarter-rows]: fp16 weights
    float2 meta[kPartGenes];          // (scale, offset) per gene of the part
    int2 stage[kWaves][2][kWave];     // per wave, two rows: (LDS byte offset of the row, value)
    int len[kWaves * kRw];            // prologue: row lengths
    std::uint32_t rows[kWaves * kRw]; // prologue: row of (wave, slot)
};

// Output column held by `lane` after reduce_scatter: 8 (lane % 8) + 4 bit3 + 2 bit4 + bit5.
__device__ __forceinline__ int scatter_column(int lane) {
    return 8 * (lane & 7) + 4 * ((lane >> 3) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 5) & 1);
}

// Sums the 8 lane groups' partials of columns 8 j + k (k < 8, j = lane % 8) and leaves
// each lane with the total of scatter_column(lane).
__device__ __forceinline__ float reduce_scatter(const float (&p)[8], int lane) {
    float q[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        // lanes 32..63 of p[2m] trade places with lanes 0..31 of p[2m+1]
        const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[2 * m]),
                                                        __float_as_uint(p[2 * m + 1]), false, false);
        q[m] = __uint_as_float(s[0]) + __uint_as_float(s[1]);  // bit5 = 0: slot 2m, 1: 2m+1
    }
    float r[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(q[2 * n]),
                                                        __float_as_uint(q[2 * n + 1]), false, false);
        r[n] = __uint_as_float(s[0]) + __uint_as_float(s[1]);  // bit4 selects q[2n + bit4]
    }
    const bool hi = (lane & 8) != 0;
    const float keep = hi ? r[1] : r[0];
    const float send = hi ? r[0] : r[1];
    // row_ror:8 inside each 16-lane row pairs lane l with l ^ 8
    const float got = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0x128, 0xf, 0xf, false));
    return keep + got;
}

// A row's register window: entries [base, base + 64) as the raw column index and the byte
// holding the entry's code (`base` - `begin` is a multiple of the codes per byte, so lane
// i's code sits at byte i / cpb, shift (i % cpb) * bits). Lanes past the row end are not
// loaded; every reader bounds the lanes by the row end.
struct Window {
    std::uint32_t col;
    std::uint32_t byte;
};

// `pb` is the packed byte of entry `base`; `entries` / `bytes` are the matrix totals. The
// loads are buffer loads from descriptors built in scalar registers with a constant lane
// offset, so they write the window registers directly (no address registers that would
// have to wait for earlier loads), and the descriptor bounds stop them at the end of the
// matrix arrays (those lanes read zeros; readers bound lanes by the row end anyway).
template<int kBits>
__device__ __forceinline__ void load_window(Window &w, const QcsrArgs &a, int base, int pb, int lane,
                                            int entries, int bytes) {
    constexpr int kCpb = 8 / kBits;
    const std::uint32_t ub = static_cast<std::uint32_t>(base), upb = static_cast<std::uint32_t>(pb);
    const std::uint32_t n = static_cast<std::uint32_t>(entries) - ub < kWave ? static_cast<std::uint32_t>(entries) - ub : kWave;
    const std::uint32_t nb = static_cast<std::uint32_t>(bytes) - upb < kWave / kCpb
        ? static_cast<std::uint32_t>(bytes) - upb : kWave / kCpb;
    const rsrc_t rc = make_rsrc(a.col_idx + ub, n * 4u);
    const rsrc_t rp = make_rsrc(a.packed + upb, nb);
    w.col = static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rc, lane * 4, 0, 0));
    w.byte = __builtin_amdgcn_raw_buffer_load_b8(rp, lane / kCpb, 0, 0);
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
    const rsrc_t rw = make_rsrc(rhs + static_cast<std::int64_t>(lo) * rhs_ld,
                                static_cast<std::uint32_t>(hi - lo - 1) * row_bytes + 128u);
#pragma unroll
    for (int k = 0; k < kChunks / kWaves; ++k) {
        const int chunk = k * kWaves + wave;
        const int idx = chunk * kWave + lane;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rw, (lds_ptr)(&w[chunk * kWave]), 16,
            static_cast<std::uint32_t>(idx / 8) * row_bytes + static_cast<std::uint32_t>(idx % 8) * 16u, 0, 0, 0);
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
            const rsrc_t rm = make_rsrc(reinterpret_cast<const float2 *>(a.scales) + lo,
                                        static_cast<std::uint32_t>(span) * 8u);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_ptr)(&sh.meta[wave * 2 * kWave]), 16,
                                                     static_cast<std::uint32_t>(wave * kWave + lane) * 16u, 0, 0, 0);
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

template<int kBits, int kPolicy, int kWaves, int kRw>
__global__ __launch_bounds__(kWaves * kWave) void qcsr_spmm_parts(QcsrArgs a) {
    constexpr int kBlockRows = kWaves * kRw;
    constexpr int kCpb = 8 / kBits;
    static_assert(kBlockRows <= kWaves * kWave && kRw <= kWave && kRw % 2 == 0, "bad part-kernel shape");
    __shared__ PartsShared<kWaves, kRw> sh;
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int grp = lane >> 3;
    const int j = lane & 7;
    const std::uint32_t first = blockIdx.x * static_cast<std::uint32_t>(kBlockRows);
    const std::uint32_t code_shift = static_cast<std::uint32_t>((lane % kCpb) * kBits);

    assign_rows<kWaves, kRw>(sh.len, sh.rows, a.row_ptr, a.rows, first, tid);

    // Matrix totals (window loads stop at them).
    const int nnz = __builtin_amdgcn_readfirstlane(a.row_ptr[a.rows]);
    const int nbytes = __builtin_amdgcn_readfirstlane(a.packed_row_ptr[a.rows]);

    // Per-row state (wave-uniform, kept in scalar registers): cursor, end, window base,
    // packed byte of the window base, row offset (column-scale/row-offset decode).
    int cur[kRw], end[kRw], base[kRw], pb[kRw];
    float roff[kRw];
    float acc[kRw][8];
    Window win[kRw];
#pragma unroll
    for (int rw = 0; rw < kRw; ++rw) {
        const std::uint32_t row = __builtin_amdgcn_readfirstlane(sh.rows[wave * kRw + rw]);
        cur[rw] = end[rw] = pb[rw] = 0;
        roff[rw] = 0.0f;
        if (row != kNoRow) {
            cur[rw] = __builtin_amdgcn_readfirstlane(a.row_ptr[row]);
            end[rw] = __builtin_amdgcn_readfirstlane(a.row_ptr[row + 1]);
            pb[rw] = __builtin_amdgcn_readfirstlane(a.packed_row_ptr[row]);
            if constexpr (kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
                roff[rw] = a.row_offsets != nullptr
                    ? __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(a.row_offsets[row])))
                    : 0.0f;
        }
        base[rw] = cur[rw];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[rw][k] = 0.0f;
        win[rw].col = kNoGene;
        win[rw].byte = 0u;
        if (cur[rw] < end[rw]) load_window<kBits>(win[rw], a, base[rw], pb[rw], lane, nnz, nbytes);
    }

    const char *wbase = reinterpret_cast<const char *>(sh.w) + j * 16;

    // Run of row rw's window lanes from the cursor whose genes lie in [lo, lo + span), cut
    // at the row end: window lanes [start, start + cnt); g = gene - lo per lane.
    auto segment = [&](int rw, int lo, std::uint32_t span, int &start, int &cnt, std::uint32_t &g) {
        start = cur[rw] - base[rw];  // 0 <= start < 64
        g = win[rw].col - static_cast<std::uint32_t>(lo);
        const std::uint64_t run = ~(__builtin_amdgcn_ballot_w64(g < span) >> start);
        const int in_run = run == 0u ? kWave - start : __builtin_ctzll(run);
        cnt = in_run < end[rw] - cur[rw] ? in_run : end[rw] - cur[rw];
    };
    // Decodes the run into stage slot `slot`: (LDS byte offset of the weight row, value).
    auto decode = [&](int rw, int slot, int start, int cnt, std::uint32_t g) {
        if (static_cast<std::uint32_t>(lane - start) < static_cast<std::uint32_t>(cnt)) {
            const float2 md = sh.meta[g];
            const float code = static_cast<float>((win[rw].byte >> code_shift) & ((1u << kBits) - 1u));
            const float off = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET ? roff[rw] : md.y;
            sh.stage[wave][slot][lane] = make_int2(static_cast<int>(g) * 128,
                                                   __float_as_int(__builtin_fmaf(code, md.x, off)));
        }
    };
    // `pairs` two-entry steps from ep, then the run's last cnt % 16 entries: lane group grp
    // takes staged entry s + grp, lane j reads 16 B of its weight row.
    auto steps = [&](int rw, const int2 *ep, int pairs, int cnt) {
        for (int k = pairs; k > 0; --k, ep += 16) {
            const int2 e0 = ep[0], e1 = ep[8];
            const uint4 w0 = *reinterpret_cast<const uint4 *>(wbase + e0.x);
            const uint4 w1 = *reinterpret_cast<const uint4 *>(wbase + e1.x);
            fma8(acc[rw], __int_as_float(e0.y), w0);
            fma8(acc[rw], __int_as_float(e1.y), w1);
        }
        if ((cnt & 8) != 0) {
            const int2 e = ep[0];
            fma8(acc[rw], __int_as_float(e.y), *reinterpret_cast<const uint4 *>(wbase + e.x));
            ep += 8;
        }
        if (grp < (cnt & 7)) {
            const int2 e = ep[0];
            fma8(acc[rw], __int_as_float(e.y), *reinterpret_cast<const uint4 *>(wbase + e.x));
        }
    };
    // Moves row rw's cursor past a run ending at window lane `stop`; when the run used the
    // window up inside the part, loads the next 64 entries and returns true.
    auto advance = [&](int rw, int stop, int cnt) -> bool {
        cur[rw] += cnt;
        if (stop < kWave || cur[rw] >= end[rw]) return false;
        base[rw] = cur[rw];
        pb[rw] += kWave / kCpb;
        load_window<kBits>(win[rw], a, base[rw], pb[rw], lane, nnz, nbytes);
        return true;
    };
    // The rest of row rw's part after a window reload, one row at a time.
    auto visit_rest = [&](int rw, int lo, std::uint32_t span) {
        for (;;) {
            int start, cnt;
            std::uint32_t g;
            segment(rw, lo, span, start, cnt, g);
            if (cnt == 0) return;
            decode(rw, 0, start, cnt, g);
            wave_sync();
            steps(rw, &sh.stage[wave][0][start + grp], cnt >> 4, cnt);
            wave_sync();
            if (!advance(rw, start + cnt, cnt)) return;
        }
    };

    // Refills row rw's window for the next part when fewer than kRefill entries are left
    // (from the cursor rounded down to a code byte). Issued right after the row's visit, the
    // loads write the window registers directly and complete behind the rest of the part.
    auto refill = [&](int rw) {
        if (base[rw] + kWave < end[rw] && base[rw] + kWave - cur[rw] < kRefill) {
            const int step = (cur[rw] - base[rw]) / kCpb;
            base[rw] += step * kCpb;
            pb[rw] += step;
            load_window<kBits>(win[rw], a, base[rw], pb[rw], lane, nnz, nbytes);
        }
    };

    const int cols = static_cast<int>(a.cols);
    const int parts = (cols + kPartGenes - 1) / kPartGenes;
    for (int part = 0; part < parts; ++part) {
        const int lo = part * kPartGenes;
        const int hi = lo + kPartGenes < cols ? lo + kPartGenes : cols;
        const std::uint32_t span = static_cast<std::uint32_t>(hi - lo);
        __syncthreads();  // every wave is done reading part - 1
        load_part<kPolicy, kWaves>(sh, a, lo, hi, wave, lane, tid);  // also completes the refills
        __syncthreads();
        // Rows are visited in pairs so two independent decode / step chains are in flight.
#pragma unroll
        for (int ra = 0; ra < kRw; ra += 2) {
            const int rb = ra + 1;
            int sa = 0, ca = 0, sb = 0, cb = 0;
            std::uint32_t ga = 0u, gb = 0u;
            if (cur[ra] < end[ra]) segment(ra, lo, span, sa, ca, ga);
            if (cur[rb] < end[rb]) segment(rb, lo, span, sb, cb, gb);
            decode(ra, 0, sa, ca, ga);
            decode(rb, 1, sb, cb, gb);
            wave_sync();
            const int2 *epa = &sh.stage[wave][0][sa + grp];
            const int2 *epb = &sh.stage[wave][1][sb + grp];
            const int ka = ca >> 4, kb = cb >> 4;
            const int kk = ka < kb ? ka : kb;
            for (int k = kk; k > 0; --k, epa += 16, epb += 16) {
                const int2 a0 = epa[0], a1 = epa[8], b0 = epb[0], b1 = epb[8];
                const uint4 wa0 = *reinterpret_cast<const uint4 *>(wbase + a0.x);
                const uint4 wa1 = *reinterpret_cast<const uint4 *>(wbase + a1.x);
                const uint4 wb0 = *reinterpret_cast<const uint4 *>(wbase + b0.x);
                const uint4 wb1 = *reinterpret_cast<const uint4 *>(wbase + b1.x);
                fma8(acc[ra], __int_as_float(a0.y), wa0);
                fma8(acc[rb], __int_as_float(b0.y), wb0);
                fma8(acc[ra], __int_as_float(a1.y), wa1);
                fma8(acc[rb], __int_as_float(b1.y), wb1);
            }
            steps(ra, epa, ka - kk, ca);
            steps(rb, epb, kb - kk, cb);
            wave_sync();
            const bool more_a = ca > 0 && advance(ra, sa + ca, ca);
            const bool more_b = cb > 0 && advance(rb, sb + cb, cb);
            if (more_a) visit_rest(ra, lo, span);
            if (more_b) visit_rest(rb, lo, span);
            refill(ra);
            refill(rb);
        }
    }

    const int col = scatter_column(lane);
#pragma unroll
    for (int rw = 0; rw < kRw; ++rw) {
        const std::uint32_t row = __builtin_amdgcn_readfirstlane(sh.rows[wave * kRw + rw]);
        if (row == kNoRow) continue;
        if (cur[rw] < end[rw]) {
            // unfinished: recompute the row on the plain path (lane = column)
            const float v = row_fallback<kBits, kPolicy>(a, row, lane);
            a.out[static_cast<std::int64_t>(row) * a.out_ld + lane] = a.ep.active ? epilogue_value(a.ep, v, row, lane) : v;
            continue;
        }
        const float v = reduce_scatter(acc[rw], lane);
        a.out[static_cast<std::int64_t>(row) * a.out_ld + col] = a.ep.active ? epilogue_value(a.ep, v, row, col) : v;
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
int launch_bits_parts(const QcsrArgs &a, hipStream_t stream) {
    constexpr int kWaves = 16, kRw = 8;
    const unsigned rows_per_block = kWaves * kRw;
    const dim3 grid((a.rows + rows_per_block - 1) / rows_per_block), block(kWaves * kWave);
    hipLaunchKernelGGL((qcsr_spmm_parts<kBits, kPolicy, kWaves, kRw>), grid, block, 0, stream, a);
    return check_launch("qcsr_spmm_parts");
}

template<int kPolicy>
int launch_policy_parts(const QcsrArgs &a, std::uint32_t bits, hipStream_t stream) {
    switch (bits) {
    case 1: return launch_bits_parts<1, kPolicy>(a, stream);
    case 2: return launch_bits_parts<2, kPolicy>(a, stream);
    case 4: return launch_bits_parts<4, kPolicy>(a, stream);
    default: return launch_bits_parts<8, kPolicy>(a, stream);
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
