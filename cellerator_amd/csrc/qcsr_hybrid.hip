// qcsr_hybrid.hip -- quantized CSR SpMM in execution order with a dense head on the matrix
// cores (fp16 weights, 64 output columns per launch).
//
// In an execution order that puts the most frequently stored genes first (the popularity
// order of exec_order.hip, or any frozen plan order), the first H genes of a single-cell
// matrix are stored in a large share of the cells: at C3, the first 4,096 of 33,538 genes
// hold 2/3 of the nonzeros at 24% mean density (59% for the first 1,024). Those columns are
// dense enough for the matrix cores. Y = X[:, 0:H) . W[0:H, :] + X[:, H:) . W[H:, :]: the
// head runs here on the matrix cores over a dense copy of X[:, 0:H); the tail runs on
// the row-group VALU kernel of qcsr_parts.hip, which starts every row at its first entry
// >= H and adds the head's sums before its epilogue.
//
// Head layout (built once per matrix by cx_qcsr_hybrid_prepare; the CSR itself is unchanged
// and still serves the tail). Word-major, row-minor arrays of rows_ld rows (rows rounded up
// to a workgroup; padding rows are zero), so the 16 rows of a matrix tile read 64
// consecutive bytes of a word:
//   codes [H * bits / 32][rows_ld] u32: word w of a row holds the codes of genes
//         [w * 32 / bits, (w + 1) * 32 / bits), gene g at bit (g % (32 / bits)) * bits;
//         zero where the row stores no such gene;
//   masks [H / 32][rows_ld] u32: bit g % 32 of word g / 32 is set where the row stores g;
//   head_end [rows]: each row's first entry whose gene is >= H (the tail's start);
//   meta [H] (scale, offset) per head gene and, for the column-scale / row-offset policy,
//         row offsets, all multiplied by 2^k (k = scale_exp).
//
// Exactness. x' = fma(code, 2^k s, 2^k o) = 2^k fma(code, s, o) exactly: the reference
// decode (include/Cellerator/quantized/access.cuh:81-91) rounds once, and scaling by a power
// of two commutes with that rounding. x' is split into three fp16 parts with
// round-toward-zero conversions, hi = rtz(x'), mid = rtz(x' - hi), lo = rtz(x' - hi - mid):
// each residual is exact in fp32 (it has at most 13, then 2, significant bits), so
// hi + mid + lo == x' whenever x' is a multiple of 2^-14 below 2^15 (every nonzero part is
// then an fp16 normal number; the matrix cores are not relied on to keep fp16 subnormal
// inputs) -- always for 2^9 <= |x'| < 2^15. k = 14 - floor(log2 B) for B the largest
// |decoded value| any head code can take, so |x'| < 2^15 and hi cannot overflow. The layout
// is refused unless every value the head can decode lies on that 2^-14 grid and splits
// exactly (head_exact_kernel, checked on the device at prepare); cx_qcsr_head_order
// (qcsr_exec.hip) picks head genes for which it does and orders the rest after the head.
// Each part times an fp16 weight is exact in fp32 and the matrix cores accumulate in fp32;
// the sums are multiplied by 2^-k (exact). The result differs from an fp32 FMA chain over the
// decoded values only in summation order.
//
// Kernel: a workgroup of 4 waves, 64 rows per wave (four 16-row tiles), no LDS. Per 32-gene
// chunk, lane (row r = lane % 16 of a tile, gene octet q = lane / 16) decodes its 8 genes
// from one code word and one mask byte straight into the three B fragments (the operand
// layout of the 16x16x32 instruction: 8 consecutive K values of one column per lane), and the
// wave issues 4 tiles x 4 column blocks x 3 parts = 48 MFMAs against A = W^T fragments read
// from the packed panel ([H/32][N][32] fp16: one coalesced kilobyte per fragment, shared by
// every wave through L2). The loads of chunk c + 1 are issued before chunk c is decoded.
// Lane l ends with output columns 4(l / 16) .. +3 of row l % 16 of each tile and column block.
#include "qcsr_common.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

typedef _Float16 cx_half8 __attribute__((ext_vector_type(8)));
typedef float cx_float4 __attribute__((ext_vector_type(4)));
typedef float cx_float16 __attribute__((ext_vector_type(16)));
typedef __fp16 cx_fp16x2 __attribute__((ext_vector_type(2)));

namespace cx {
namespace {

constexpr int kHeadWaves = 4;
constexpr int kTiles = 4;                             // 16-row tiles per wave
constexpr int kRowsPerWave = 16 * kTiles;
constexpr std::uint32_t kHeadRows = kHeadWaves * kRowsPerWave;  // rows per workgroup
constexpr std::uint32_t kHeadAlign = 1024;            // head_cols granularity (the tail's gene part)

struct HeadArgs {
    const std::uint32_t *codes;
    const std::uint32_t *masks;
    const float2 *meta;          // [head] pre-scaled (scale, offset)
    const float *row_offsets;    // [rows] pre-scaled (column-scale / row-offset policy), else null
    const std::uint16_t *panel;  // fp16 [head/32][panel_n][32] at this launch's first column
    float *partial;              // [rows][64] fp32: Y_head
    std::uint32_t rows;
    std::uint32_t rows_ld;
    std::uint32_t chunks;        // head / 32
    std::uint32_t panel_n;
    float inv_scale;
    std::uint64_t part_stride;   // floats between the partials of two gene parts (grid.y > 1)             // 2^-k
};

template<int kBits>
struct CodeWords {
    std::uint32_t w[kBits == 8 ? 2 : 1];
};

template<int kBits>
__device__ __forceinline__ CodeWords<kBits> load_code_words(const HeadArgs &h, std::uint32_t c, int q,
                                                            std::uint32_t row) {
    CodeWords<kBits> cw;
    if constexpr (kBits == 8) {
        const std::uint32_t *p = h.codes + static_cast<std::uint64_t>(c * 8u + 2u * q) * h.rows_ld + row;
        cw.w[0] = p[0];
        cw.w[1] = p[h.rows_ld];
    } else {
        // octet q covers bits [8 q bits, 8 q bits + 8 bits) of the chunk's `bits` words
        cw.w[0] = h.codes[static_cast<std::uint64_t>(c * kBits + (q * kBits) / 4) * h.rows_ld + row];
    }
    return cw;
}

// Sign-extended bit j of v (0 or all ones), kept as one v_bfe_i32: the AND-mask form of a
// presence bit, which the optimizer would otherwise rewrite into a compare and a select.
template<int kBit>
__device__ __forceinline__ std::uint32_t bit_mask(std::uint32_t v) {
    std::uint32_t r;
    asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(r) : "v"(v), "n"(kBit));
    return r;
}

// Byte k of v as a float, one v_cvt_f32_ubyte<k> (the optimizer would otherwise extract
// the byte with a shift or a bitfield extract first).
template<int kByte>
__device__ __forceinline__ float ubyte_f32(std::uint32_t v) {
    float r;
    if constexpr (kByte == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (kByte == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (kByte == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// x - float(half kHalf of h2), exact (x - rtz(x) fits in fp32), as one v_fma_mix_f32 that
// widens the fp16 operand itself (the optimizer would split it into a conversion and a
// subtraction).
template<int kHalf>
__device__ __forceinline__ float sub_half(float x, std::uint32_t h2) {
    float r;
    if constexpr (kHalf == 0) asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(x));
    else asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(x));
    return r;
}

// Code of gene j of an octet as a float: 4- and 8-bit codes through byte conversions.
template<int kBits, int kJ>
__device__ __forceinline__ float octet_code(const std::uint32_t (&w)[2], std::uint32_t lo4, std::uint32_t hi4) {
    if constexpr (kBits == 8) return ubyte_f32<kJ & 3>(w[kJ >> 2]);
    else if constexpr (kBits == 4) return ubyte_f32<(kJ >> 1)>((kJ & 1) != 0 ? hi4 : lo4);
    else return static_cast<float>((w[0] >> (kJ * kBits)) & ((1u << kBits) - 1u));
}

// fp16 parts of a pair of values: rtz conversions, each residual one v_fma_mix_f32.
__device__ __forceinline__ void split_pair(float x0, float x1, std::uint32_t &hw, std::uint32_t &mw, std::uint32_t &lw) {
    hw = __builtin_bit_cast(std::uint32_t, __builtin_amdgcn_cvt_pkrtz(x0, x1));
    const float r0 = sub_half<0>(x0, hw);
    const float r1 = sub_half<1>(x1, hw);
    mw = __builtin_bit_cast(std::uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
    lw = __builtin_bit_cast(std::uint32_t, __builtin_amdgcn_cvt_pkrtz(sub_half<0>(r0, mw), sub_half<1>(r1, mw)));
}

template<int kBits, int kPolicy, int kJ>
__device__ __forceinline__ float octet_value(const std::uint32_t (&w)[2], std::uint32_t lo4, std::uint32_t hi4,
                                             std::uint32_t mb, const float2 (&md)[8], float roff) {
    const float off = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET ? roff : md[kJ].y;
    const float v = __builtin_fmaf(octet_code<kBits, kJ>(w, lo4, hi4), md[kJ].x, off);
    return __uint_as_float(__float_as_uint(v) & bit_mask<kJ>(mb));  // absent genes: +0
}

// The 8 genes of one octet, decoded, masked and split into three fp16 fragments.
template<int kBits, int kPolicy>
__device__ __forceinline__ void decode_octet(const CodeWords<kBits> &cw, int q, std::uint32_t mask_word,
                                             const float2 (&md)[8], float roff, cx_half8 &bh, cx_half8 &bm,
                                             cx_half8 &bl) {
    const std::uint32_t mb = mask_word >> (8 * q);
    std::uint32_t w[2] = {cw.w[0], kBits == 8 ? cw.w[kBits == 8 ? 1 : 0] : 0u};
    if constexpr (kBits < 8) w[0] = cw.w[0] >> ((8 * q * kBits) & 31);
    const std::uint32_t lo4 = w[0] & 0x0f0f0f0fu;
    const std::uint32_t hi4 = (w[0] >> 4) & 0x0f0f0f0fu;
    std::uint32_t hw[4], mw[4], lw[4];
    split_pair(octet_value<kBits, kPolicy, 0>(w, lo4, hi4, mb, md, roff),
               octet_value<kBits, kPolicy, 1>(w, lo4, hi4, mb, md, roff), hw[0], mw[0], lw[0]);
    split_pair(octet_value<kBits, kPolicy, 2>(w, lo4, hi4, mb, md, roff),
               octet_value<kBits, kPolicy, 3>(w, lo4, hi4, mb, md, roff), hw[1], mw[1], lw[1]);
    split_pair(octet_value<kBits, kPolicy, 4>(w, lo4, hi4, mb, md, roff),
               octet_value<kBits, kPolicy, 5>(w, lo4, hi4, mb, md, roff), hw[2], mw[2], lw[2]);
    split_pair(octet_value<kBits, kPolicy, 6>(w, lo4, hi4, mb, md, roff),
               octet_value<kBits, kPolicy, 7>(w, lo4, hi4, mb, md, roff), hw[3], mw[3], lw[3]);
    bh = __builtin_bit_cast(cx_half8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
    bm = __builtin_bit_cast(cx_half8, make_uint4(mw[0], mw[1], mw[2], mw[3]));
    bl = __builtin_bit_cast(cx_half8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
}

template<int kBits>
struct ChunkLoads {
    cx_half8 aw[4];             // A = W^T fragments of the 4 column blocks
    float2 md[8];               // pre-scaled (scale, offset) of the octet's genes
    CodeWords<kBits> cw[kTiles];
    std::uint32_t mw[kTiles];
};

template<int kBits>
__device__ __forceinline__ void load_chunk(ChunkLoads<kBits> &L, const HeadArgs &h, std::uint32_t c, int q, int r16,
                                           std::uint32_t row0) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
        L.aw[t] = *reinterpret_cast<const cx_half8 *>(
            h.panel + (static_cast<std::uint64_t>(c) * h.panel_n + t * 16 + r16) * 32u + 8u * q);
    const float4 *mp = reinterpret_cast<const float4 *>(h.meta + c * 32u + 8u * q);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 v = mp[k];
        L.md[2 * k] = make_float2(v.x, v.y);
        L.md[2 * k + 1] = make_float2(v.z, v.w);
    }
    const std::uint32_t *mrow = h.masks + static_cast<std::uint64_t>(c) * h.rows_ld;
#pragma unroll
    for (int b = 0; b < kTiles; ++b) {
        const std::uint32_t row = row0 + 16u * b;
        L.mw[b] = mrow[row];
        L.cw[b] = load_code_words<kBits>(h, c, q, row);
    }
}

template<int kBits, int kPolicy>
__global__ __launch_bounds__(kHeadWaves * kWave) void qcsr_head_dense(HeadArgs h) {
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int r16 = lane & 15;
    const int q = lane >> 4;
    // row of tile 0 (tile b: + 16 b); rows up to rows_ld exist in the dense arrays
    const std::uint32_t row0 = blockIdx.x * kHeadRows + static_cast<std::uint32_t>(wave * kRowsPerWave + r16);

    float roff[kTiles];
#pragma unroll
    for (int b = 0; b < kTiles; ++b) {
        const std::uint32_t row = row0 + 16u * b;
        roff[b] = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET && h.row_offsets != nullptr && row < h.rows
            ? h.row_offsets[row] : 0.0f;
    }

    cx_float4 acc[kTiles][4];
#pragma unroll
    for (int b = 0; b < kTiles; ++b)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[b][t] = cx_float4{0.0f, 0.0f, 0.0f, 0.0f};

    auto chunk = [&](const ChunkLoads<kBits> &L) {
#pragma unroll
        for (int b = 0; b < kTiles; ++b) {
            cx_half8 bh, bm, bl;
            decode_octet<kBits, kPolicy>(L.cw[b], q, L.mw[b], L.md, roff[b], bh, bm, bl);
            // each accumulator's three products are 4 instructions apart
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(L.aw[t], bh, acc[b][t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(L.aw[t], bm, acc[b][t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(L.aw[t], bl, acc[b][t], 0, 0, 0);
        }
    };
    // gene part blockIdx.y of gridDim.y: chunks [c_begin, c_end), its own partial
    const std::uint32_t c_begin = blockIdx.y * h.chunks / gridDim.y, c_end = (blockIdx.y + 1u) * h.chunks / gridDim.y;
    float *partial = h.partial + blockIdx.y * h.part_stride;
    ChunkLoads<kBits> cur, nxt;
    if (c_begin < c_end) load_chunk<kBits>(cur, h, c_begin, q, r16, row0);
    for (std::uint32_t c = c_begin; c < c_end; ++c) {
        if (c + 1u < c_end) load_chunk<kBits>(nxt, h, c + 1u, q, r16, row0);
        chunk(cur);
        cur = nxt;
    }

#pragma unroll
    for (int b = 0; b < kTiles; ++b) {
        const std::uint32_t row = row0 + 16u * b;
        if (row < h.rows) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float *o = partial + static_cast<std::uint64_t>(row) * 64u + t * 16 + 4 * q;
                *reinterpret_cast<float4 *>(o) = make_float4(acc[b][t][0] * h.inv_scale, acc[b][t][1] * h.inv_scale,
                                                             acc[b][t][2] * h.inv_scale, acc[b][t][3] * h.inv_scale);
            }
        }
    }
}

// ---- the table form: code bytes and a per-gene table of pre-split values -------------------
//
// For codes of up to 4 bits under a per-gene decode policy, the 17 values a head gene can take
// (codes 0..15, and "not stored") are split once, at prepare, into their three fp16 parts:
// lut[chunk][gene][code] = (hi, mid, lo, 0), entry 16 all zero. The head plane then holds one
// byte per (row, gene), code * 8 or 128 when the gene is not stored (the table entry's byte
// offset), chunk-major: bytes[chunk][rows_ld][32]. Decoding a value is one table read; the
// parts of two genes are packed into the fragments with byte permutes. The values are those
// of the per-value decode above; the products run on v_mfma_f32_32x32x16_f16 (two 32-row
// tiles x two 32-column tiles per wave), so they are summed in another order.
//
// Workgroup: 4 waves of 64 rows. Per 32-gene chunk the W^T fragments (4 KB, in fragment order),
// the chunk's table (4,352 B) and the workgroup's code bytes (8 KB) go through an LDS double
// buffer, loaded straight into LDS while the previous chunk is computed; one barrier per
// chunk. No registers hold the share, so the kernel fits four waves per SIMD.

constexpr int kLutWaves = 4;
constexpr std::uint32_t kLutRows = kLutWaves * kRowsPerWave;  // 256 rows per workgroup
constexpr std::uint32_t kLayoutRows = 512;                    // row granularity of the head planes
constexpr std::uint32_t kLutEntries = 17;                     // codes 0..15 and "not stored"
constexpr std::uint32_t kLutGeneBytes = kLutEntries * 8u;     // 136
constexpr std::uint32_t kLutChunkBytes = 32u * kLutGeneBytes; // 4,352
constexpr std::uint32_t kCodeChunkBytes = kLutRows * 32u;     // the workgroup's code bytes of one chunk
static_assert(kLayoutRows % kLutRows == 0u && kLayoutRows % kHeadRows == 0u, "head plane rows");
constexpr std::uint32_t kAbsentWord = 0x80808080u;            // four genes not stored: entry 16 (byte 128)

struct LutArgs {
    const std::uint8_t *bytes;   // [head/32][rows_ld][32]
    const uint4 *lut;            // [head/32][kLutChunkBytes / 16]
    const std::uint16_t *panel;  // fp16 [head/32][panel_n][32] at this launch's first column
    float *partial;              // [rows][64] fp32: Y_head
    std::uint32_t rows;
    std::uint32_t rows_ld;
    std::uint32_t chunks;
    std::uint32_t panel_n;
    float inv_scale;
};

struct LutShared {
    uint4 a[2][4][kWave];                  // W^T fragments: [buffer][K step * 2 + column tile][lane]
    uint4 lut[2][kLutChunkBytes / 16];     // the chunk's table
    uint4 codes[2][kCodeChunkBytes / 16];  // the workgroup's code bytes: [row][32]
};

typedef unsigned int head_rsrc_t __attribute__((ext_vector_type(4)));

// Buffer resource over [base, base + bytes): loads past the end return 0.
__device__ __forceinline__ head_rsrc_t head_rsrc(const void *base, std::uint32_t bytes) {
    const std::uint64_t a = reinterpret_cast<std::uint64_t>(base);
    head_rsrc_t r;
    r.x = static_cast<unsigned int>(a);
    r.y = static_cast<unsigned int>(a >> 32) & 0xffffu;  // stride 0
    r.z = bytes;
    r.w = 0x00020000u;
    return r;
}

// 16 bytes per lane from the buffer at voffset straight into LDS at dst + 16 * lane (a buffer
// load with the lds flag; the LDS address is taken from m0 when the load issues). Issued as
// inline assembly so that the compiler sees no LDS write: as a builtin it would wait for
// every such load before any later LDS read it cannot tell apart from the loaded buffer
// (both buffers are one array indexed at run time), and the prefetch of the next chunk
// would stop overlapping the current one (measured: 615 against 571 us per launch at C3).
// The kernel waits for these loads itself (vmcnt) before the barrier that publishes a
// buffer. m0 is saved and restored around the load, so the statement leaves every register
// the compiler owns as it was.
__device__ __forceinline__ void lds_load16(head_rsrc_t rsrc, const void *dst, std::uint32_t voffset) {
    using lds_ptr = const __attribute__((address_space(3))) char *;
    const std::uint32_t base = static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>((lds_ptr)dst));
    std::uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %1\n\t"
                 "s_nop 0\n\t"
                 "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(base), "v"(voffset), "s"(rsrc)
                 : "memory");
}

// The share of chunk c goes straight from memory into LDS buffer `buf` (buffer loads with the
// lds flag: each wave instruction fills 1 KB, no registers): the A fragments (wave w loads
// fragment (K step w / 2, column tile w % 2): lane l reads row 32 (w % 2) + l % 32 of the
// panel, genes 16 (l / 32) + 8 (w / 2) .. +7), table pieces w * 64 + lane (pieces 256..271
// by lanes 0..15 of wave 0), and the workgroup's code bytes, pieces w * 64 + lane and
// 256 + w * 64 + lane.
__device__ __forceinline__ void issue_share(LutShared &sh, const LutArgs &h, std::uint32_t c, int buf, int wave,
                                            int lane, std::uint32_t wg_row) {
    const head_rsrc_t pa = head_rsrc(h.panel + static_cast<std::uint64_t>(c) * h.panel_n * 32u, 64u * 64u);
    const std::uint32_t uw = static_cast<std::uint32_t>(wave), ul = static_cast<std::uint32_t>(lane);
    const std::uint32_t pa_off = ((32u * (uw % 2u) + ul % 32u) * 32u + 16u * (ul / 32u) + 8u * (uw / 2u)) * 2u;
    lds_load16(pa, &sh.a[buf][wave][0], pa_off);
    const head_rsrc_t lu = head_rsrc(h.lut + static_cast<std::uint64_t>(c) * (kLutChunkBytes / 16u), kLutChunkBytes);
    const std::uint32_t piece = uw * kWave + ul;
    lds_load16(lu, &sh.lut[buf][wave * kWave], piece * 16u);
    const head_rsrc_t cb = head_rsrc(h.bytes + (static_cast<std::uint64_t>(c) * h.rows_ld + wg_row) * 32u, kCodeChunkBytes);
    lds_load16(cb, &sh.codes[buf][wave * kWave], piece * 16u);
    lds_load16(cb, &sh.codes[buf][256 + wave * kWave], (256u + piece) * 16u);
    if (wave == 0 && lane < static_cast<int>(kLutChunkBytes / 16u) - 256)
        lds_load16(lu, &sh.lut[buf][256], (256u + ul) * 16u);
}

static_assert(kLutWaves * kWave == 256 && kCodeChunkBytes / 16u == 512u && kLutChunkBytes / 16u == 272u, "share pieces");

// Byte k of v as a 32-bit offset.
template<int kK>
__device__ __forceinline__ std::uint32_t byte_of(std::uint32_t v) {
    return kK == 3 ? v >> 24 : (v >> (8 * kK)) & 0xffu;
}

// Table entries of the 8 genes gene0 .. gene0 + 7 (from the chunk table at lb) for the code
// bytes in w0 (genes 0..3) and w1 (genes 4..7), packed into the three B fragments.
__device__ __forceinline__ void lut_fragments(const char *lb, std::uint32_t w0, std::uint32_t w1, cx_half8 &bh,
                                              cx_half8 &bm, cx_half8 &bl) {
    uint2 e[8];
    e[0] = *reinterpret_cast<const uint2 *>(lb + 0 * kLutGeneBytes + byte_of<0>(w0));
    e[1] = *reinterpret_cast<const uint2 *>(lb + 1 * kLutGeneBytes + byte_of<1>(w0));
    e[2] = *reinterpret_cast<const uint2 *>(lb + 2 * kLutGeneBytes + byte_of<2>(w0));
    e[3] = *reinterpret_cast<const uint2 *>(lb + 3 * kLutGeneBytes + byte_of<3>(w0));
    e[4] = *reinterpret_cast<const uint2 *>(lb + 4 * kLutGeneBytes + byte_of<0>(w1));
    e[5] = *reinterpret_cast<const uint2 *>(lb + 5 * kLutGeneBytes + byte_of<1>(w1));
    e[6] = *reinterpret_cast<const uint2 *>(lb + 6 * kLutGeneBytes + byte_of<2>(w1));
    e[7] = *reinterpret_cast<const uint2 *>(lb + 7 * kLutGeneBytes + byte_of<3>(w1));
    std::uint32_t hw[4], mw[4], lw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // (hi | mid << 16, lo) of genes 2k and 2k + 1 -> hi pair, mid pair, lo pair
        hw[k] = __builtin_amdgcn_perm(e[2 * k + 1].x, e[2 * k].x, 0x05040100u);
        mw[k] = __builtin_amdgcn_perm(e[2 * k + 1].x, e[2 * k].x, 0x07060302u);
        lw[k] = __builtin_amdgcn_perm(e[2 * k + 1].y, e[2 * k].y, 0x05040100u);
    }
    bh = __builtin_bit_cast(cx_half8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
    bm = __builtin_bit_cast(cx_half8, make_uint4(mw[0], mw[1], mw[2], mw[3]));
    bl = __builtin_bit_cast(cx_half8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
}

// v_mfma_f32_32x32x16_f16 with A = W^T (32 output columns x 16 genes) and B = the decoded
// parts (16 genes x 32 rows). The chunk's 32 genes are two K steps; lane half hf carries
// genes 16 hf .. 16 hf + 15 (K step ks: 16 hf + 8 ks .. +7) in both operands, so its 32
// lanes read one gene's table at a time. A wave holds 2 row tiles x 2 column tiles; each
// part's four products are independent, so an accumulator is reused every fourth
// instruction, which keeps the 16-pass instruction at full rate.
__global__ __launch_bounds__(kLutWaves * kWave) __attribute__((amdgpu_waves_per_eu(4, 4))) void qcsr_head_lut(LutArgs h) {
    __shared__ LutShared sh;
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int r32 = lane & 31;
    const int hf = lane >> 5;
    const std::uint32_t wg_row = blockIdx.x * kLutRows;
    const std::uint32_t row0 = wg_row + static_cast<std::uint32_t>(wave * kRowsPerWave + r32);
    cx_float16 acc[2][2];  // [row tile][column tile]
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rt][ct][i] = 0.0f;

    if (h.chunks != 0u) issue_share(sh, h, 0u, 0, wave, lane, wg_row);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's share loads are in LDS
    __syncthreads();
    for (std::uint32_t c = 0; c < h.chunks; ++c) {
        const int buf = static_cast<int>(c & 1u);
        // chunk c + 1 into the buffer chunk c - 1 used (every wave passed the barrier after it)
        if (c + 1u < h.chunks) issue_share(sh, h, c + 1u, buf ^ 1, wave, lane, wg_row);
        const char *lb = reinterpret_cast<const char *>(&sh.lut[buf][0]) + 16u * hf * kLutGeneBytes;
        const char *cbase = reinterpret_cast<const char *>(&sh.codes[buf][0]) + (wave * kRowsPerWave + r32) * 32 + 16 * hf;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const cx_half8 a0 = __builtin_bit_cast(cx_half8, sh.a[buf][2 * ks][lane]);
            const cx_half8 a1 = __builtin_bit_cast(cx_half8, sh.a[buf][2 * ks + 1][lane]);
            cx_half8 bh[2], bm[2], bl[2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const uint2 cw = *reinterpret_cast<const uint2 *>(cbase + 32 * 32 * rt + 8 * ks);
                lut_fragments(lb + 8 * ks * kLutGeneBytes, cw.x, cw.y, bh[rt], bm[rt], bl[rt]);
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                acc[rt][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bh[rt], acc[rt][0], 0, 0, 0);
                acc[rt][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bh[rt], acc[rt][1], 0, 0, 0);
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                acc[rt][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bm[rt], acc[rt][0], 0, 0, 0);
                acc[rt][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bm[rt], acc[rt][1], 0, 0, 0);
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                acc[rt][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bl[rt], acc[rt][0], 0, 0, 0);
                acc[rt][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bl[rt], acc[rt][1], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's loads of chunk c + 1 are in LDS
        __syncthreads();  // buffer `buf` is free again; chunk c + 1 is in place
    }

    // lane l holds row l % 32 of each row tile; register 4j + i is output column
    // 32 ct + 8j + 4 (l / 32) + i
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const std::uint32_t row = row0 + 32u * rt;
        if (row < h.rows) {
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float *o = h.partial + static_cast<std::uint64_t>(row) * 64u + ct * 32 + 8 * j + 4 * hf;
                    *reinterpret_cast<float4 *>(o) =
                        make_float4(acc[rt][ct][4 * j] * h.inv_scale, acc[rt][ct][4 * j + 1] * h.inv_scale,
                                    acc[rt][ct][4 * j + 2] * h.inv_scale, acc[rt][ct][4 * j + 3] * h.inv_scale);
                }
        }
    }
}

// ---- building the dense head -----------------------------------------------------------

struct BuildArgs {
    const std::int32_t *row_ptr;
    const std::int32_t *packed_row_ptr;
    const std::int32_t *col_idx;
    const std::uint8_t *packed;
    std::uint32_t rows;
    std::uint32_t rows_ld;
    std::uint32_t head;
    std::uint32_t *codes;
    std::uint32_t *masks;
    std::int32_t *head_end;
    std::uint32_t *error;  // set to 1 where a row's genes are not strictly increasing
};

// One thread per row (consecutive rows in consecutive lanes, so every word store of a
// wave is 256 contiguous bytes): walks the row's head entries in order and writes every
// code word and mask word of the row, zeros included.
template<int kBits>
__global__ __launch_bounds__(256) void dense_head_build(BuildArgs a) {
    const std::uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= a.rows_ld) return;
    constexpr std::uint32_t kGenesPerWord = 32u / kBits;
    constexpr std::uint32_t kMask = (1u << kBits) - 1u;
    const std::uint32_t words = a.head / kGenesPerWord;
    std::int64_t e = 0, end = 0, rb = 0, pbit = 0;
    if (row < a.rows) {
        rb = e = a.row_ptr[row];
        end = a.row_ptr[row + 1];
        pbit = static_cast<std::int64_t>(a.packed_row_ptr[row]) * 8;
    }
    std::int64_t prev = -1;
    bool bad = false;
    std::uint32_t mword = 0u;
    for (std::uint32_t w = 0; w < words; ++w) {
        const std::int64_t g_lo = static_cast<std::int64_t>(w) * kGenesPerWord;
        const std::int64_t g_hi = g_lo + kGenesPerWord;
        std::uint32_t word = 0u;
        while (e < end) {
            const std::int64_t c = a.col_idx[e];
            if (c >= g_hi) break;
            if (c <= prev) {  // repeated, decreasing or negative gene: not a sorted row
                bad = true;
                break;
            }
            const std::int64_t bit = pbit + (e - rb) * kBits;
            const std::uint32_t code = (static_cast<std::uint32_t>(a.packed[bit >> 3]) >> (bit & 7)) & kMask;
            word |= code << (static_cast<std::uint32_t>(c - g_lo) * kBits);
            mword |= 1u << (static_cast<std::uint32_t>(c) & 31u);
            prev = c;
            ++e;
        }
        a.codes[static_cast<std::uint64_t>(w) * a.rows_ld + row] = word;
        if (((w + 1u) * kGenesPerWord) % 32u == 0u) {
            a.masks[static_cast<std::uint64_t>((w + 1u) * kGenesPerWord / 32u - 1u) * a.rows_ld + row] = mword;
            mword = 0u;
        }
        if (bad) e = end;  // the remaining words of the row stay zero
    }
    if (row < a.rows) a.head_end[row] = static_cast<std::int32_t>(e);
    if (bad) atomicOr(a.error, 1u);
}

// Table form: one wave per row (kBytesRowsPerWave consecutive rows per wave) reads the row's
// head entries 64 at a time, coalesced, and drops each code byte (code * 8) into an LDS copy
// of 64 chunks x 32 bytes preset to 128 ("not stored"); lane c then stores chunk c's 32 bytes
// as two 16-byte writes. Also the row's first tail entry. A row whose head genes are not
// strictly increasing and non-negative keeps the bytes of the entries before the first bad
// one, its later chunks stay "not stored", its first tail entry is its end, and the error
// word is set.
constexpr int kBytesWaves = 4;
constexpr std::uint32_t kBytesRowsPerWave = 16;
constexpr std::uint32_t kBytesRows = kBytesWaves * kBytesRowsPerWave;  // rows per workgroup
static_assert(kLayoutRows % kBytesRows == 0u, "head plane rows");

template<int kBits>
__global__ __launch_bounds__(kBytesWaves * kWave) void dense_head_bytes(BuildArgs a, std::uint8_t *bytes) {
    constexpr std::uint32_t kMask = (1u << kBits) - 1u;
    __shared__ std::uint32_t plane[kBytesWaves][kWave * 8];  // per wave: 64 chunks of 32 bytes
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    std::uint8_t *pb = reinterpret_cast<std::uint8_t *>(plane[wave]);
    auto lds_order = [] { __asm__ volatile("" ::: "memory"); };
    const std::uint32_t chunks = a.head / 32u;
    for (std::uint32_t r = 0; r < kBytesRowsPerWave; ++r) {
        const std::uint32_t row = (blockIdx.x * kBytesWaves + static_cast<std::uint32_t>(wave)) * kBytesRowsPerWave + r;
        if (row >= a.rows_ld) break;
        std::int64_t e = 0, end = 0, rb = 0, pbit = 0;
        if (row < a.rows) {
            rb = e = __builtin_amdgcn_readfirstlane(a.row_ptr[row]);
            end = __builtin_amdgcn_readfirstlane(a.row_ptr[row + 1]);
            pbit = static_cast<std::int64_t>(__builtin_amdgcn_readfirstlane(a.packed_row_ptr[row])) * 8;
        }
        std::int64_t prev = -1;
        bool bad = false;
        for (std::uint32_t c0 = 0; c0 < chunks; c0 += kWave) {
            lds_order();
#pragma unroll
            for (int d = 0; d < 8; ++d) plane[wave][lane * 8 + d] = kAbsentWord;
            lds_order();
            const std::int64_t g_lo = static_cast<std::int64_t>(c0) * 32;
            const std::int64_t g_hi = static_cast<std::int64_t>(min(c0 + kWave, chunks)) * 32;
            while (e < end) {
                const std::int64_t idx = e + lane;
                const bool valid = idx < end;
                const std::int64_t gene = valid ? static_cast<std::int64_t>(a.col_idx[idx]) : g_hi;
                std::int64_t before = static_cast<std::int64_t>(__shfl_up(static_cast<int>(gene), 1, kWave));
                if (lane == 0) before = prev;
                const bool in = valid && gene < g_hi;
                const std::uint64_t bad_lanes = __builtin_amdgcn_ballot_w64(in && gene <= before);
                const std::uint64_t in_lanes = __builtin_amdgcn_ballot_w64(in);
                // sorted rows: the chunk window's entries are a prefix of the lanes
                const int first_bad = bad_lanes != 0u ? __builtin_ctzll(bad_lanes) : kWave;
                const std::uint64_t ok = in_lanes & (first_bad == kWave ? ~std::uint64_t{0} : (std::uint64_t{1} << first_bad) - 1u);
                if (((ok >> lane) & 1u) != 0u) {
                    const std::int64_t bit = pbit + (idx - rb) * kBits;
                    const std::uint32_t code = (static_cast<std::uint32_t>(a.packed[bit >> 3]) >> (bit & 7)) & kMask;
                    pb[gene - g_lo] = static_cast<std::uint8_t>(code * 8u);
                }
                if (bad_lanes != 0u) {
                    bad = true;
                    break;
                }
                const int n = __popcll(in_lanes);
                if (n > 0) prev = static_cast<std::int64_t>(__builtin_amdgcn_readlane(static_cast<int>(gene), n - 1));
                e += n;
                if (n < kWave) break;
            }
            lds_order();
            if (c0 + static_cast<std::uint32_t>(lane) < chunks) {
                uint4 *dst = reinterpret_cast<uint4 *>(bytes + (static_cast<std::uint64_t>(c0 + lane) * a.rows_ld + row) * 32u);
                const std::uint32_t *src = &plane[wave][lane * 8];
                dst[0] = make_uint4(src[0], src[1], src[2], src[3]);
                dst[1] = make_uint4(src[4], src[5], src[6], src[7]);
            }
            if (bad) e = end;  // the remaining chunks of the row stay "not stored"
        }
        if (lane == 0) {
            if (row < a.rows) a.head_end[row] = static_cast<std::int32_t>(e);
            if (bad) atomicOr(a.error, 1u);
        }
    }
}

// lut[chunk][gene][code] = the three round-toward-zero fp16 parts of fma(code, 2^k s, 2^k o)
// (the per-value decode's split, computed once) for codes up to qmax; other entries (codes
// the width cannot hold, and entry 16) zero.
__global__ __launch_bounds__(256) void head_lut_kernel(const float2 *meta, std::uint32_t head, std::uint32_t qmax,
                                                       std::uint16_t *lut) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= head * kLutEntries) return;
    const std::uint32_t g = i / kLutEntries, code = i % kLutEntries;
    std::uint32_t hw = 0u, mw = 0u, lw = 0u;
    if (code <= qmax) {
        const float2 md = meta[g];
        split_pair(__builtin_fmaf(static_cast<float>(code), md.x, md.y), 0.0f, hw, mw, lw);
    }
    std::uint16_t *dst = lut + ((g / 32u) * kLutChunkBytes + (g % 32u) * kLutGeneBytes + code * 8u) / 2u;
    dst[0] = static_cast<std::uint16_t>(hw & 0xffffu);
    dst[1] = static_cast<std::uint16_t>(mw & 0xffffu);
    dst[2] = static_cast<std::uint16_t>(lw & 0xffffu);
    dst[3] = 0u;
}

// Largest |decoded value| any code of a head gene can take, as float bits (non-negative
// floats order like their bit patterns): per-gene affine max(|o|, |o + qmax s|); column
// scale with row offsets |s| qmax (the row offsets' largest magnitude is found separately).
__global__ __launch_bounds__(256) void head_range_kernel(const float *scales, const float *offsets, std::uint32_t policy,
                                                         std::uint32_t head, float qmax, std::uint32_t *max_bits) {
    const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    float b = 0.0f;
    if (g < head) {
        float s, o;
        if (policy == CX_DECODE_PER_GENE_AFFINE_PAIRS) {
            s = scales[2 * g];
            o = scales[2 * g + 1];
        } else {
            s = scales != nullptr ? scales[g] : 1.0f;
            o = policy == CX_DECODE_PER_GENE_AFFINE && offsets != nullptr ? offsets[g] : 0.0f;
        }
        b = fmaxf(fabsf(o), fabsf(__builtin_fmaf(qmax, s, o)));
        if (policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET) b = fabsf(s) * qmax;
        if (!(s == s) || !(o == o) || !(b == b)) b = __builtin_huge_valf();  // NaN metadata: reject
    }
    for (int d = 32; d >= 1; d >>= 1) b = fmaxf(b, __shfl_xor(b, d, kWave));
    if ((threadIdx.x & (kWave - 1)) == 0) atomicMax(max_bits, __float_as_uint(b));
}

__global__ __launch_bounds__(256) void abs_max_kernel(const float *v, std::uint32_t n, std::uint32_t *max_bits) {
    float b = 0.0f;
    for (std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float a = fabsf(v[i]);
        b = fmaxf(b, a == a ? a : __builtin_huge_valf());
    }
    for (int d = 32; d >= 1; d >>= 1) b = fmaxf(b, __shfl_xor(b, d, kWave));
    if ((threadIdx.x & (kWave - 1)) == 0) atomicMax(max_bits, __float_as_uint(b));
}

// Scaling by 2^k kept the value: no rounding, and the result is zero or a normal float.
__device__ __forceinline__ bool exactly_scaled(float scaled, float value, float inv) {
    const float a = fabsf(scaled);
    return scaled * inv == value && a < __builtin_huge_valf() && (a == 0.0f || a >= 0x1p-126f);
}

// A scaled value the three fp16 parts can carry: a multiple of 2^-14 below 2^15.
__device__ __forceinline__ bool on_head_grid(float x) {
    const float t = x * 16384.0f;
    return fabsf(x) < 32768.0f && t == truncf(t);
}

__device__ __forceinline__ bool normal_or_zero_half(std::uint32_t h) {
    return (h & 0x7fffu) == 0u || ((h >> 10) & 0x1fu) != 0u;
}

// Exactness of the head under the layout scale 2^k (factor = 2^k, inv = 2^-k). Per-gene
// policies, one thread per (head gene g, code c): x' = fma(c, 2^k s, 2^k o) must equal
// 2^k fma(c, s, o), lie on the 2^-14 grid below 2^15, and split into three parts that are zero
// or fp16 normal numbers summing to x'. Row-offset policy, one thread per head gene: 2^k s
// exactly scaled and on the grid; with every 2^k r on the grid too (head_exact_rows_kernel),
// each fma(c, 2^k s, 2^k r) is (the exact sum is a multiple of 2^-14 and rounding to fp32
// keeps that), and the layout bound keeps it below 2^15. A failing gene g records g + 1.
__global__ __launch_bounds__(256) void head_exact_kernel(const float *scales, const float *offsets, std::uint32_t policy,
                                                         std::uint32_t head, std::uint32_t codes, float factor,
                                                         float inv, std::uint32_t *bad) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= head * codes) return;
    const std::uint32_t g = i / codes, c = i % codes;
    float s, o;
    if (policy == CX_DECODE_PER_GENE_AFFINE_PAIRS) {
        s = scales[2 * g];
        o = scales[2 * g + 1];
    } else {
        s = scales != nullptr ? scales[g] : 1.0f;
        o = policy == CX_DECODE_PER_GENE_AFFINE && offsets != nullptr ? offsets[g] : 0.0f;
    }
    const float s2 = s * factor, o2 = o * factor;
    bool ok = exactly_scaled(s2, s, inv) && exactly_scaled(o2, o, inv);
    if (policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET) {
        ok = ok && on_head_grid(s2);
    } else if (ok) {
        const float x2 = __builtin_fmaf(static_cast<float>(c), s2, o2);
        ok = x2 * inv == __builtin_fmaf(static_cast<float>(c), s, o) && on_head_grid(x2);
        if (ok) {
            std::uint32_t hw, mw, lw;
            split_pair(x2, 0.0f, hw, mw, lw);
            ok = normal_or_zero_half(hw) && normal_or_zero_half(mw) && normal_or_zero_half(lw)
                 && static_cast<double>(h2f(hw & 0xffffu)) + static_cast<double>(h2f(mw & 0xffffu))
                            + static_cast<double>(h2f(lw & 0xffffu)) == static_cast<double>(x2);
        }
    }
    if (!ok) atomicMax(bad, g + 1u);
}

// Row-offset policy: every 2^k r exactly scaled and on the 2^-14 grid; a failing row records
// row + 1.
__global__ __launch_bounds__(256) void head_exact_rows_kernel(const float *row_offsets, std::uint32_t rows,
                                                              float factor, float inv, std::uint32_t *bad) {
    for (std::uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x) {
        const float v = row_offsets[r], v2 = v * factor;
        if (!(exactly_scaled(v2, v, inv) && on_head_grid(v2))) atomicMax(bad, r + 1u);
    }
}

__global__ void zero_words(std::uint32_t *p, int n) {
    if (static_cast<int>(threadIdx.x) < n) p[threadIdx.x] = 0u;
}

// meta[g] = 2^k (scale, offset) of head gene g (offset 0 under the row-offset policy);
// row_offsets_out[r] = 2^k row offset.
__global__ __launch_bounds__(256) void scale_meta_kernel(const float *scales, const float *offsets,
                                                         const float *row_offsets, std::uint32_t policy,
                                                         std::uint32_t head, std::uint32_t rows, float factor,
                                                         float2 *meta, float *row_offsets_out) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < head) {
        float s, o;
        if (policy == CX_DECODE_PER_GENE_AFFINE_PAIRS) {
            s = scales[2 * i];
            o = scales[2 * i + 1];
        } else {
            s = scales != nullptr ? scales[i] : 1.0f;
            o = policy == CX_DECODE_PER_GENE_AFFINE && offsets != nullptr ? offsets[i] : 0.0f;
        }
        meta[i] = make_float2(s * factor, o * factor);
    }
    if (row_offsets_out != nullptr && i < rows)
        row_offsets_out[i] = row_offsets != nullptr ? row_offsets[i] * factor : 0.0f;
}

bool valid_bits(std::uint32_t b) { return b == 1u || b == 2u || b == 4u || b == 8u; }

int validate_hybrid(const cx_qcsr_matrix *m, std::uint32_t head, const char *who) {
    if (m == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, who);
    if (!valid_bits(m->bits))
        return fail(CX_STATUS_UNSUPPORTED, "hybrid quantized CSR: codes of 1, 2, 4 or 8 bits only");
    if (m->decode_policy != CX_DECODE_PER_GENE_AFFINE && m->decode_policy != CX_DECODE_PER_GENE_AFFINE_PAIRS
        && m->decode_policy != CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
        return fail(CX_STATUS_UNSUPPORTED, "hybrid quantized CSR: unknown decode policy");
    if (head % kHeadAlign != 0u || head > m->cols)
        return fail(CX_STATUS_INVALID_SHAPE, "hybrid quantized CSR: head_cols must be a multiple of 1,024 within cols");
    if (m->rows != 0u && (m->row_ptr == nullptr || m->packed_row_ptr == nullptr
                          || (m->nnz != 0u && (m->col_idx == nullptr || m->packed_values == nullptr))))
        return fail(CX_STATUS_INVALID_ARGUMENT, "hybrid quantized CSR: null structure or codes");
    if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS && m->column_scales == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "hybrid quantized CSR: the pairs policy needs column_scales");
    if ((m->flags & CX_QCSR_COLUMNS_SORTED) == 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "hybrid quantized CSR: rows must be sorted (CX_QCSR_COLUMNS_SORTED, e.g. from cx_qcsr_to_execution_order)");
    if (m->nnz > static_cast<std::uint64_t>(INT32_MAX) || m->cols > static_cast<std::uint32_t>(INT32_MAX))
        return fail(CX_STATUS_INVALID_SHAPE, "hybrid quantized CSR: nnz exceeds int32 row offsets");
    return CX_STATUS_SUCCESS;
}

constexpr std::uint64_t align256(std::uint64_t b) { return (b + 255u) & ~std::uint64_t{255u}; }

// Table form for codes of up to 4 bits under a per-gene policy; code words and presence bits
// otherwise (8-bit codes have 257 table entries per gene; row offsets make a value depend on
// the row).
std::uint32_t head_form(const cx_qcsr_matrix *m) {
    return m->bits <= 4u && m->decode_policy != CX_DECODE_COLUMN_SCALE_ROW_OFFSET ? CX_HEAD_FORM_TABLE
                                                                                  : CX_HEAD_FORM_WORDS;
}

struct LayoutSizes {
    std::uint64_t header, codes, masks, bytes, lut, head_end, meta, row_offsets, total;
    std::uint32_t rows_ld, form;
};

LayoutSizes layout_sizes(const cx_qcsr_matrix *m, std::uint32_t head) {
    LayoutSizes s{};
    s.form = head_form(m);
    s.rows_ld = static_cast<std::uint32_t>((static_cast<std::uint64_t>(m->rows) + kLayoutRows - 1) / kLayoutRows * kLayoutRows);
    s.header = 256;
    if (s.form == CX_HEAD_FORM_WORDS) {
        s.codes = align256(static_cast<std::uint64_t>(head) * m->bits / 32u * s.rows_ld * 4u);
        s.masks = align256(static_cast<std::uint64_t>(head) / 32u * s.rows_ld * 4u);
    } else {
        s.bytes = align256(static_cast<std::uint64_t>(head) * s.rows_ld);
        s.lut = align256(static_cast<std::uint64_t>(head) / 32u * kLutChunkBytes);
    }
    s.head_end = align256(static_cast<std::uint64_t>(m->rows) * 4u);
    s.meta = align256(static_cast<std::uint64_t>(head) * 8u);
    s.row_offsets = m->decode_policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET ? align256(static_cast<std::uint64_t>(m->rows) * 4u) : 0u;
    s.total = s.header + s.codes + s.masks + s.bytes + s.lut + s.head_end + s.meta + s.row_offsets;
    return s;
}

// Launches the dense head kernel for one 64-column block.
// Gene parts of the words-form head: its waves cover 64 rows each, so a matrix with fewer
// than four such waves per SIMD splits the head's genes into up to three parts, one partial
// each (summed in order by the tail), to give every SIMD several waves. The table form, and
// any head of larger matrices, runs in one part.
std::uint32_t head_parts(std::uint32_t form, std::uint32_t rows_ld, std::uint32_t head_cols) {
    if (form != CX_HEAD_FORM_WORDS || head_cols == 0u) return 1u;
    const std::uint64_t waves = rows_ld / static_cast<std::uint64_t>(kRowsPerWave);
    const std::uint64_t simds = 4ull * blocks_per_round();
    if (waves == 0u || waves >= 4u * simds) return 1u;
    const std::uint64_t want = (4u * simds + waves - 1u) / waves;
    return static_cast<std::uint32_t>(std::min<std::uint64_t>({want, 3u, head_cols / 32u}));
}

std::uint64_t partial_stride_floats(std::uint32_t rows) {
    return align256(static_cast<std::uint64_t>(rows) * 64u * 4u) / 4u;
}

int launch_head(const cx_qcsr_hybrid_layout &L, const std::uint16_t *panel, std::uint32_t panel_n, float *partial,
                hipStream_t stream) {
    if (L.head_form == CX_HEAD_FORM_TABLE) {
        LutArgs t{};
        t.bytes = L.code_bytes;
        t.lut = reinterpret_cast<const uint4 *>(L.lut);
        t.panel = panel;
        t.partial = partial;
        t.rows = L.rows;
        t.rows_ld = L.rows_ld;
        t.chunks = L.head_cols / 32u;
        t.panel_n = panel_n;
        t.inv_scale = std::ldexp(1.0f, -L.scale_exp);
        hipLaunchKernelGGL(qcsr_head_lut, dim3(L.rows_ld / kLutRows), dim3(kLutWaves * kWave), 0, stream, t);
        return check_launch("qcsr_head_lut");
    }
    HeadArgs h{};
    h.codes = L.codes;
    h.masks = L.masks;
    h.meta = reinterpret_cast<const float2 *>(L.meta);
    h.row_offsets = L.row_offsets;
    h.panel = panel;
    h.partial = partial;
    h.rows = L.rows;
    h.rows_ld = L.rows_ld;
    h.chunks = L.head_cols / 32u;
    h.panel_n = panel_n;
    h.inv_scale = std::ldexp(1.0f, -L.scale_exp);
    h.part_stride = partial_stride_floats(L.rows);
    const dim3 grid(L.rows_ld / kHeadRows, head_parts(L.head_form, L.rows_ld, L.head_cols)), block(kHeadWaves * kWave);
#define CX_HEAD(B, P) hipLaunchKernelGGL((qcsr_head_dense<B, P>), grid, block, 0, stream, h)
#define CX_HEAD_POLICY(B)                                                                        \
    do {                                                                                         \
        if (L.decode_policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET) CX_HEAD(B, CX_DECODE_COLUMN_SCALE_ROW_OFFSET); \
        else CX_HEAD(B, CX_DECODE_PER_GENE_AFFINE);                                              \
    } while (0)
    switch (L.bits) {
    case 1: CX_HEAD_POLICY(1); break;
    case 2: CX_HEAD_POLICY(2); break;
    case 4: CX_HEAD_POLICY(4); break;
    default: CX_HEAD_POLICY(8); break;
    }
#undef CX_HEAD_POLICY
#undef CX_HEAD
    return check_launch("qcsr_head_dense");
}

} // namespace

int head_scale_exp(float total) {
    int k = 0;
    if (total > 0.0f) {
        int ex = 0;
        (void)std::frexp(total, &ex);  // total = f 2^ex, f in [0.5, 1): floor(log2) = ex - 1
        k = 14 - (ex - 1);
    }
    return std::max(-100, std::min(100, k));
}

} // namespace cx

extern "C" int cx_qcsr_hybrid_layout_bytes(const cx_qcsr_matrix *m, uint32_t head_cols, uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (bytes == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_hybrid_layout_bytes: null bytes");
    const int rc = validate_hybrid(m, head_cols, "cx_qcsr_hybrid_layout_bytes: null matrix");
    if (rc != CX_STATUS_SUCCESS) return rc;
    *bytes = layout_sizes(m, head_cols).total;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_hybrid_prepare(const cx_qcsr_matrix *m, uint32_t head_cols, void *storage,
                                      uint64_t storage_bytes, cx_qcsr_hybrid_layout *layout, void *stream) {
    using namespace cx;
    clear_error();
    int rc = validate_hybrid(m, head_cols, "cx_qcsr_hybrid_prepare: null matrix");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (layout == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_hybrid_prepare: null layout");
    const LayoutSizes sz = layout_sizes(m, head_cols);
    if (storage == nullptr || storage_bytes < sz.total || (reinterpret_cast<std::uintptr_t>(storage) & 255u) != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_hybrid_prepare: storage must be 256-byte aligned and hold cx_qcsr_hybrid_layout_bytes");
    cx_qcsr_hybrid_layout L{};
    L.head_cols = head_cols;
    L.rows = m->rows;
    L.rows_ld = sz.rows_ld;
    L.bits = m->bits;
    L.decode_policy = m->decode_policy;
    L.nnz = m->nnz;
    L.head_form = sz.form;
    auto *base = static_cast<unsigned char *>(storage);
    std::uint64_t off = sz.header;
    if (sz.form == CX_HEAD_FORM_WORDS) {
        L.codes = reinterpret_cast<uint32_t *>(base + off);
        off += sz.codes;
        L.masks = reinterpret_cast<uint32_t *>(base + off);
        off += sz.masks;
    } else {
        L.code_bytes = reinterpret_cast<uint8_t *>(base + off);
        off += sz.bytes;
        L.lut = reinterpret_cast<uint16_t *>(base + off);
        off += sz.lut;
    }
    L.head_end = reinterpret_cast<int32_t *>(base + off);
    off += sz.head_end;
    L.meta = reinterpret_cast<float *>(base + off);
    off += sz.meta;
    L.row_offsets = sz.row_offsets != 0u ? reinterpret_cast<float *>(base + off) : nullptr;

    const hipStream_t s = static_cast<hipStream_t>(stream);
    auto *words = reinterpret_cast<std::uint32_t *>(base);  // header: range bits, row-offset bits, error
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, s, words, 6);
    if (head_cols != 0u) {
        const float qmax = static_cast<float>((1u << m->bits) - 1u);
        hipLaunchKernelGGL(head_range_kernel, dim3((head_cols + 255u) / 256u), dim3(256), 0, s, m->column_scales,
                           m->column_offsets, m->decode_policy, head_cols, qmax, words);
        if (m->decode_policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET && m->row_offsets != nullptr && m->rows != 0u)
            hipLaunchKernelGGL(abs_max_kernel, dim3(std::min<std::uint32_t>((m->rows + 255u) / 256u, 4096u)), dim3(256),
                               0, s, m->row_offsets, m->rows, words + 1);
    }
    if (L.rows_ld != 0u) {
        BuildArgs b{};
        b.row_ptr = m->row_ptr;
        b.packed_row_ptr = m->packed_row_ptr;
        b.col_idx = m->col_idx;
        b.packed = m->packed_values;
        b.rows = m->rows;
        b.rows_ld = L.rows_ld;
        b.head = head_cols;
        b.codes = L.codes;
        b.masks = L.masks;
        b.head_end = L.head_end;
        b.error = words + 2;
        const dim3 grid(L.rows_ld / 256u), block(256);
        if (sz.form == CX_HEAD_FORM_TABLE) {
            const dim3 tgrid(L.rows_ld / kBytesRows), tblock(kBytesWaves * kWave);
            switch (m->bits) {
            case 1: hipLaunchKernelGGL(dense_head_bytes<1>, tgrid, tblock, 0, s, b, L.code_bytes); break;
            case 2: hipLaunchKernelGGL(dense_head_bytes<2>, tgrid, tblock, 0, s, b, L.code_bytes); break;
            default: hipLaunchKernelGGL(dense_head_bytes<4>, tgrid, tblock, 0, s, b, L.code_bytes); break;
            }
        } else {
            switch (m->bits) {
            case 1: hipLaunchKernelGGL(dense_head_build<1>, grid, block, 0, s, b); break;
            case 2: hipLaunchKernelGGL(dense_head_build<2>, grid, block, 0, s, b); break;
            case 4: hipLaunchKernelGGL(dense_head_build<4>, grid, block, 0, s, b); break;
            default: hipLaunchKernelGGL(dense_head_build<8>, grid, block, 0, s, b); break;
            }
        }
    }
    rc = check_launch("cx_qcsr_hybrid_prepare");
    if (rc != CX_STATUS_SUCCESS) return rc;
    std::uint32_t host[4] = {0u, 0u, 0u, 0u};
    hipError_t e = hipMemcpyAsync(host, words, sizeof(host), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "cx_qcsr_hybrid_prepare");
    if (host[2] != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_hybrid_prepare: a row's genes are not strictly increasing despite CX_QCSR_COLUMNS_SORTED");
    float bound, roff;
    std::memcpy(&bound, &host[0], 4);
    std::memcpy(&roff, &host[1], 4);
    const float total = bound + roff;
    if (!(total < 3.0e38f))
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_hybrid_prepare: head metadata is not finite");
    const int k = head_scale_exp(total);
    if (!(std::ldexp(total, k) < 32768.0f))
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_hybrid_prepare: head values of 2^115 or more");
    L.scale_exp = k;
    const std::uint32_t n = std::max(head_cols, L.row_offsets != nullptr ? m->rows : 0u);
    if (n != 0u) {
        hipLaunchKernelGGL(scale_meta_kernel, dim3((n + 255u) / 256u), dim3(256), 0, s, m->column_scales,
                           m->column_offsets, m->row_offsets, m->decode_policy, head_cols, m->rows,
                           std::ldexp(1.0f, k), reinterpret_cast<float2 *>(L.meta), L.row_offsets);
        rc = check_launch("cx_qcsr_hybrid_prepare");
        if (rc != CX_STATUS_SUCCESS) return rc;
    }
    if (sz.form == CX_HEAD_FORM_TABLE && head_cols != 0u) {
        hipLaunchKernelGGL(head_lut_kernel, dim3((head_cols * kLutEntries + 255u) / 256u), dim3(256), 0, s,
                           reinterpret_cast<const float2 *>(L.meta), head_cols, (1u << m->bits) - 1u, L.lut);
        rc = check_launch("cx_qcsr_hybrid_prepare");
        if (rc != CX_STATUS_SUCCESS) return rc;
    }
    if (head_cols != 0u) {
        // every value the head can decode must be carried exactly by its fp16 parts
        const bool row_policy = m->decode_policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET;
        const std::uint32_t codes = row_policy ? 1u : (1u << m->bits);
        const float factor = std::ldexp(1.0f, k), inv = std::ldexp(1.0f, -k);
        hipLaunchKernelGGL(head_exact_kernel, dim3((head_cols * codes + 255u) / 256u), dim3(256), 0, s,
                           m->column_scales, m->column_offsets, m->decode_policy, head_cols, codes, factor, inv,
                           words + 4);
        if (row_policy && m->row_offsets != nullptr)
            hipLaunchKernelGGL(head_exact_rows_kernel, dim3(std::min<std::uint32_t>((m->rows + 255u) / 256u, 4096u)),
                               dim3(256), 0, s, m->row_offsets, m->rows, factor, inv, words + 5);
        rc = check_launch("cx_qcsr_hybrid_prepare");
        if (rc != CX_STATUS_SUCCESS) return rc;
        std::uint32_t bad[2] = {0u, 0u};
        e = hipMemcpyAsync(bad, words + 4, sizeof(bad), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) return hip_fail(e, "cx_qcsr_hybrid_prepare");
        if (bad[0] != 0u) {
            set_error("cx_qcsr_hybrid_prepare: head gene %u does not decode exactly under the layout scale 2^%d "
                      "(cx_qcsr_head_order places such genes after the head)", bad[0] - 1u, k);
            return CX_STATUS_UNSUPPORTED;
        }
        if (bad[1] != 0u) {
            set_error("cx_qcsr_hybrid_prepare: the offset of row %u does not decode exactly under the layout scale "
                      "2^%d (under the row-offset policy every row offset must; cx_qcsr_head_order then gives no head)",
                      bad[1] - 1u, k);
            return CX_STATUS_UNSUPPORTED;
        }
    }
    *layout = L;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_hybrid_workspace(const cx_qcsr_matrix *m, uint32_t head_cols, int64_t out_cols,
                                        uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (m == nullptr || bytes == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_hybrid_workspace: null argument");
    if (out_cols <= 0 || out_cols % 64 != 0 || out_cols > 256)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_hybrid_workspace: out_cols must be 64, 128, 192 or 256");
    const std::uint64_t partial = partial_stride_floats(m->rows) * 4u
        * head_parts(head_form(m), layout_sizes(m, head_cols).rows_ld, head_cols);
    const std::uint64_t panel = align256(static_cast<std::uint64_t>(head_cols) * static_cast<std::uint64_t>(out_cols) * 2u);
    *bytes = partial + panel;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_spmm_fwd_hybrid(const cx_qcsr_matrix *m, const cx_qcsr_hybrid_layout *layout,
                                       const void *rhs, int64_t rhs_ld, int64_t out_cols, float *out,
                                       int64_t out_ld, const cx_spmm_epilogue *epilogue, void *workspace,
                                       uint64_t workspace_bytes, void *stream) {
    using namespace cx;
    clear_error();
    if (layout == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_hybrid: null layout");
    const cx_qcsr_hybrid_layout &L = *layout;
    int rc = validate_hybrid(m, L.head_cols, "cx_qcsr_spmm_fwd_hybrid: null matrix");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (L.rows != m->rows || L.bits != m->bits || L.decode_policy != m->decode_policy || L.nnz != m->nnz
        || L.rows_ld != layout_sizes(m, L.head_cols).rows_ld || L.head_form != head_form(m) || L.head_end == nullptr
        || (L.head_cols != 0u && (L.meta == nullptr
                                  || (L.head_form == CX_HEAD_FORM_WORDS ? L.codes == nullptr || L.masks == nullptr
                                                                        : L.code_bytes == nullptr || L.lut == nullptr))))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_hybrid: the layout was not prepared for this matrix");
    if (rhs == nullptr || out == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_hybrid: null rhs or output");
    if (out_cols <= 0 || out_cols % 64 != 0 || out_cols > 256 || rhs_ld < out_cols || out_ld < out_cols)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_fwd_hybrid: out_cols must be 64, 128, 192 or 256");
    const bool aligned = (reinterpret_cast<std::uintptr_t>(rhs) & 15u) == 0u
        && (reinterpret_cast<std::uintptr_t>(out) & 15u) == 0u && (rhs_ld * 2) % 16 == 0 && (out_ld * 4) % 16 == 0;
    if (!aligned)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_hybrid: rhs and output must be 16-byte aligned");
    if (rhs_ld > (INT32_MAX / 2) / 1024)
        return fail(CX_STATUS_INVALID_SHAPE,
                    "cx_qcsr_spmm_fwd_hybrid: rhs_ld too large (a 1,024-gene part must span under 1 GiB of W)");
    if (static_cast<const void *>(out) == rhs)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_hybrid: output aliases the rhs");
    return launch_hybrid(*m, L, rhs, rhs_ld, out_cols, out, out_ld, epilogue, workspace, workspace_bytes,
                         static_cast<hipStream_t>(stream), "cx_qcsr_spmm_fwd_hybrid");
}

namespace cx {

// The launch behind cx_qcsr_spmm_fwd_hybrid, after its checks of the matrix, layout and
// operands. From `m` it reads the shape, code width, decode policy, flags and metadata; the
// structure arrays only when the layout has no tail stream.
int launch_hybrid(const cx_qcsr_matrix &mm, const cx_qcsr_hybrid_layout &L, const void *rhs, std::int64_t rhs_ld,
                  std::int64_t out_cols, float *out, std::int64_t out_ld, const cx_spmm_epilogue *epilogue,
                  void *workspace, std::uint64_t workspace_bytes, hipStream_t s, const char *who) {
    const cx_qcsr_matrix *m = &mm;
    int rc = CX_STATUS_SUCCESS;
    if (m->rows == 0u) return CX_STATUS_SUCCESS;
    Epilogue ep;
    rc = make_epilogue(epilogue, m->rows, out_cols, out, out_ld, &ep, who);
    if (rc != CX_STATUS_SUCCESS) return rc;
    std::uint64_t need = 0u;
    (void)cx_qcsr_hybrid_workspace(m, L.head_cols, out_cols, &need);
    if (L.head_cols != 0u && (workspace == nullptr || workspace_bytes < need
                              || (reinterpret_cast<std::uintptr_t>(workspace) & 255u) != 0u))
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_spmm_fwd_hybrid: needs a 256-byte aligned workspace of cx_qcsr_hybrid_workspace bytes");
    QcsrArgs a{};
    a.ep = ep;
    a.row_ptr = m->row_ptr;
    a.packed_row_ptr = m->packed_row_ptr;
    a.col_idx = m->col_idx;
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
    a.flags = m->flags;
    const cx_qcsr_tail_stream *ts = L.tail;
    if (ts != nullptr) {
        const std::uint32_t all_parts = (m->cols + kHeadAlign - 1u) / kHeadAlign;
        if (ts->rows != m->rows || ts->bits != m->bits || ts->nnz != m->nnz || ts->first_part != L.head_cols / kHeadAlign
            || ts->parts != all_parts - ts->first_part
            || ts->blocks < (std::uint64_t{m->rows} + kStreamRows - 1u) / kStreamRows
            || ts->blocks > (std::uint64_t{m->rows} + 7u) / 8u
            || ts->block_rows != kStreamRows || ts->layers != kStreamLayers
            || ts->slot_rows == nullptr || ts->fill_index == nullptr || ts->entries == nullptr)
            return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_hybrid: the tail stream was not built for this layout");
        a.slot_rows = ts->slot_rows;
        a.fill_index = ts->fill_index;
        a.stream_entries = ts->entries;
        a.stream_parts = ts->parts;
        a.stream_blocks = ts->blocks;
        a.first_part = ts->first_part;
    }
    // one 64-column block of the tail: the prepared stream, else the row-group kernel
    auto tail = [&](const QcsrArgs &b) {
        return ts != nullptr ? launch_qcsr_stream(b, m->bits, m->decode_policy, s)
                             : launch_qcsr_parts(b, m->bits, m->decode_policy, 64, s);
    };
    if (L.head_cols == 0u) {
        if (ts == nullptr) return launch_qcsr_parts(a, m->bits, m->decode_policy, out_cols, s);
        for (std::int64_t c0 = 0; c0 < out_cols; c0 += 64) {
            QcsrArgs b = a;
            b.rhs = static_cast<const std::uint16_t *>(rhs) + c0;
            b.out = out + c0;
            if (b.ep.bias != nullptr) b.ep.bias += c0;
            if (b.ep.initial != nullptr) b.ep.initial += c0;
            rc = tail(b);
            if (rc != CX_STATUS_SUCCESS) return rc;
        }
        return CX_STATUS_SUCCESS;
    }
    auto *partial = static_cast<float *>(workspace);
    const std::uint32_t hparts = head_parts(L.head_form, L.rows_ld, L.head_cols);
    auto *panel = reinterpret_cast<std::uint16_t *>(static_cast<unsigned char *>(workspace)
                                                    + partial_stride_floats(m->rows) * 4u * hparts);
    // the head genes' weights as the matrix-core operand panel [H/32][out_cols][32]
    rc = pack_panel_columns(static_cast<const std::uint16_t *>(rhs), rhs_ld, L.head_cols,
                            static_cast<std::uint32_t>(out_cols), panel, s);
    if (rc != CX_STATUS_SUCCESS) return rc;
    for (std::int64_t c0 = 0; c0 < out_cols; c0 += 64) {
        rc = launch_head(L, panel + c0 * 32, static_cast<std::uint32_t>(out_cols), partial, s);
        if (rc != CX_STATUS_SUCCESS) return rc;
        QcsrArgs b = a;
        b.rhs = static_cast<const std::uint16_t *>(rhs) + c0;
        b.out = out + c0;
        if (b.ep.bias != nullptr) b.ep.bias += c0;
        if (b.ep.initial != nullptr) b.ep.initial += c0;
        b.row_start = L.head_end;
        b.acc_init = partial;
        b.acc_parts = hparts;
        b.acc_part_stride = partial_stride_floats(m->rows);
        b.first_part = L.head_cols / kHeadAlign;
        rc = tail(b);
        if (rc != CX_STATUS_SUCCESS) return rc;
    }
    return CX_STATUS_SUCCESS;
}

} // namespace cx
