// qcsr_common.hpp -- the quantized CSR operand as the kernels see it, and its decode.
#pragma once

#include "cx_common.hpp"

namespace cx {

enum class ValueMode : int { quantized = 0, f16 = 1, f32 = 2 };

struct QcsrArgs {
    const std::int32_t *row_ptr;
    const std::int32_t *packed_row_ptr;
    const std::int32_t *col_idx;
    const std::uint8_t *packed;
    const float *scales;
    const float *offsets;
    const float *row_offsets;
    const void *values;
    const void *rhs;
    std::int64_t rhs_ld;
    float *out;
    std::int64_t out_ld;
    std::uint32_t rows;
    std::uint32_t cols;
    std::uint32_t flags;  // cx_qcsr_matrix.flags (CX_QCSR_COLUMNS_SORTED)
    Epilogue ep;
    // Tail of the execution-order hybrid (row-group kernel only; NULL / 0 otherwise): each
    // row starts at entry row_start[row] instead of row_ptr[row], its sums start from
    // acc_init[row][0..64) (the head's partial), and the gene parts start at first_part.
    const std::int32_t *row_start;
    const float *acc_init;
    std::uint32_t first_part;
    // The head may leave its sums as acc_parts partials (the genes split in order), acc_init
    // + k * acc_part_stride floats; the row's sums start from their sum in that order.
    std::uint32_t acc_parts;        // 0 or 1: one partial
    std::uint64_t acc_part_stride;
    // Prepared tail stream (qcsr_spmm_stream only; built by qcsr_stream.hip): the row of
    // every (block, wave, layer, group) slot, the fill index, the entries in fill order, the
    // number of gene parts the stream covers (from first_part on) and its block count.
    const std::uint32_t *slot_rows;
    const std::uint32_t *fill_index;
    const void *stream_entries;
    std::uint32_t stream_parts;
    std::uint32_t stream_blocks;
};

// Geometry of the prepared tail stream, shared by its builder and its kernel: 16 waves of
// 8 layers of 8 rows per 1,024-row block; a fill is 16 steps of the 8 lane groups of a
// layer, 128 entries stored group-major ([group][step]); entries are u16
// (gene in part | code << 11) for codes of up to 4 bits and u32 (gene | code << 16) for
// 8-bit codes. fill_index[((block * kStreamWaves + wave) * parts + part) * kStreamLayers +
// layer] holds the layer's first fill (low 28 bits) and the step count of its last fill
// minus one (high 4 bits); the entry after the last is the total. A wave's fills are
// contiguous through all parts. Block rows are sets of 8 rows adjacent in the order of tail
// lengths over the whole matrix, dealt round-robin to the blocks (slot_rows maps every slot
// to its row).
constexpr int kStreamWaves = 16;
constexpr int kStreamLayers = 8;
constexpr int kStreamSlots = kStreamWaves * kStreamLayers;        // (wave, layer) per block and part
constexpr int kStreamRows = kStreamSlots * 8;

// Workgroups of a row-group walk over `rows` rows, each at most `max_rows` rows and at least
// one set of 8 (any count in [ceil(rows / max_rows), ceil(rows / 8)] is a valid geometry).
// When ceil(rows / max_rows) full workgroups would not fill one round of `units` (one per
// compute unit at a time), the rows are spread over `units` workgroups: 100k rows keep all
// 256 CUs busy instead of 98. Beyond that, `whole_rounds` rounds the count up to whole
// rounds (the canonical kernel's 1M rows: 2,048 workgroups of ~488 rows instead of 1,954
// full ones, measured 3% faster); otherwise the fewest full workgroups are kept (the tail
// walk's 977 blocks ran 1% faster than 1,024 smaller ones: the dispatcher balances the
// partial last round better than equal rounds do).
inline std::uint32_t round_block_count(std::uint32_t rows, std::uint32_t max_rows, std::uint32_t units,
                                       bool whole_rounds) {
    const std::uint32_t need = static_cast<std::uint32_t>((static_cast<std::uint64_t>(rows) + max_rows - 1) / max_rows);
    const std::uint32_t sets = static_cast<std::uint32_t>((static_cast<std::uint64_t>(rows) + 7) / 8);
    if (units == 0u || need == 0u || (need >= units && !whole_rounds)) return need;
    const std::uint64_t blocks = (static_cast<std::uint64_t>(need) + units - 1u) / units * units;
    return blocks < sets ? static_cast<std::uint32_t>(blocks) : sets;
}

// Workgroups per round: the environment's CX_BLOCKS_PER_ROUND when it is a positive integer
// (1 gives the fewest full workgroups), else the current device's compute units (0 when the
// query fails).
std::uint32_t blocks_per_round();
constexpr std::uint32_t kFillMask = 0x0fffffffu;
constexpr int kStreamPartGenes = 1024;
constexpr std::uint32_t kStreamPad = 1024u;                       // gene of a pad entry: a zero row
// Pads of odd parity (a second zero row): a pad takes the parity opposite to the entry of
// the paired lane group at the same step, so the two reads stay in different LDS bank halves.
constexpr std::uint32_t kStreamPadOdd = 1025u;

// One 64-column block of the tail through the prepared stream (fp16 weights).
int launch_qcsr_stream(const QcsrArgs &a, std::uint32_t bits, std::uint32_t policy, hipStream_t stream);

// The launch of cx_qcsr_spmm_fwd_hybrid once its operands are checked (qcsr_hybrid.hip): reads
// the shape, code width, decode policy, flags and metadata of `m`, its structure arrays only
// when the layout has no tail stream.
int launch_hybrid(const cx_qcsr_matrix &m, const cx_qcsr_hybrid_layout &layout, const void *rhs, std::int64_t rhs_ld,
                  std::int64_t out_cols, float *out, std::int64_t out_ld, const cx_spmm_epilogue *epilogue,
                  void *workspace, std::uint64_t workspace_bytes, hipStream_t stream, const char *who);

// The matrix-core head's scale exponent (qcsr_hybrid.hip): k = 14 - floor(log2 total), total =
// the largest |decoded value| of the head's genes plus, under the row-offset policy, the
// largest |row offset|, so every scaled value 2^k x stays below 2^15; 0 for total = 0;
// clamped to [-100, 100]. The head layout and the head order that picks its genes share it.
int head_scale_exp(float total);

constexpr int kWavesPerBlock = 4;

// Decoded value of entry `i` (global nnz index) of row `row` whose packed codes start
// at `pbase`. Returns the gene through `col`.
template<int kBits, int kPolicy, ValueMode kMode>
__device__ __forceinline__ float load_entry(const QcsrArgs &a, std::int64_t i,
                                            std::int64_t begin, const std::uint8_t *pbase,
                                            float row_offset, int &col) {
    col = a.col_idx[i];
    if constexpr (kMode == ValueMode::quantized) {
        constexpr int kCpb = 8 / kBits;
        constexpr unsigned kMask = (1u << kBits) - 1u;
        const std::int64_t local = i - begin;
        const unsigned byte = pbase[local / kCpb];
        const unsigned code = (byte >> (static_cast<unsigned>(local % kCpb) * kBits)) & kMask;
        if constexpr (kPolicy == CX_DECODE_PER_GENE_AFFINE_PAIRS) {
            // interleaved (scale, offset): one 8-byte gather
            const float2 so = reinterpret_cast<const float2 *>(a.scales)[col];
            return __builtin_fmaf(static_cast<float>(code), so.x, so.y);
        } else {
            const float scale = a.scales != nullptr ? a.scales[col] : 1.0f;
            const float offset = kPolicy == CX_DECODE_PER_GENE_AFFINE
                ? (a.offsets != nullptr ? a.offsets[col] : 0.0f)
                : row_offset;
            return __builtin_fmaf(static_cast<float>(code), scale, offset);
        }
    } else if constexpr (kMode == ValueMode::f16) {
        return h2f(static_cast<const std::uint16_t *>(a.values)[i]);
    } else {
        return static_cast<const float *>(a.values)[i];
    }
}

// Row-group kernel over LDS gene parts (qcsr_parts.hip): quantized codes, fp16 weights, N a
// multiple of 64 up to 256 (one launch per 64 columns), 16-byte aligned operands.
bool qcsr_parts_applicable(const QcsrArgs &a, std::uint32_t bits, std::uint32_t rhs_dtype,
                           std::int64_t out_cols, bool aligned);
int launch_qcsr_parts(const QcsrArgs &a, std::uint32_t bits, std::uint32_t policy, std::int64_t out_cols,
                      hipStream_t stream);
// grad_values of the backward pass by gene part (fp16 weights, N = 64).
bool bwd_values_parts_applicable(std::uint32_t rows, std::uint32_t cols, std::uint32_t rhs_dtype,
                                 std::int64_t out_cols, bool aligned, std::int64_t rhs_ld);
int launch_bwd_values_parts(const std::int32_t *row_ptr, const std::int32_t *col_idx, const float *grad_out,
                            std::int64_t grad_out_ld, const void *rhs, std::int64_t rhs_ld,
                            float *grad_values, std::uint32_t rows, std::uint32_t cols, bool sorted,
                            hipStream_t stream);

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

} // namespace cx
