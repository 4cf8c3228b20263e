// qcsr_spmm.hip -- quantized CSR SpMM on gfx950: Y = decode(X) . W, fp32 accumulate.
//
// Semantics (parity contract): each stored code is decoded exactly as the reference
// codec does, value = fma(float(code), scale, offset) with one rounding
// (include/Cellerator/quantized/access.cuh:81-91, numeric.cuh:34-36); the fp16 weight is
// widened exactly; products and sums are fp32, as csr_spmm_fwd_kernel_ computes them
// (src/compute/sparse/project/kernels/csr_spmm_fwd_kernel_.cuh:13-19) but in a fixed
// per-row order of our own (partial sums per lane group, then a butterfly).
//
// Layout of the fast path ("row per wavefront, lanes over output columns"):
//   * one wave64 owns one cell row;
//   * the row's entries are streamed 64 at a time: lane i loads col_idx[i] and its
//     code (coalesced), decodes it in registers with the per-gene scale/offset, and
//     stages (gene, value) in LDS;
//   * the wave then consumes the staged entries kEps at a time: lane group g takes
//     entry s + g, each of its kLpe lanes loads 16 B of that gene's weight row
//     (8 fp16 or 4 fp32 output columns) and issues fused multiply-adds
//     (v_fma_mix_f32 for fp16 weights: widening folded into the FMA);
//   * at the end of the row the kEps group partials are summed with a xor butterfly
//     and group 0 writes the row's N outputs (one 16/32 B store per lane).
// Any other shape (N not 32/64/128, unaligned operands) takes the generic kernel: one
// wave per row, lanes over output columns, entries in nnz order.
#include "qcsr_common.hpp"

#include <mutex>

namespace cx {
namespace {

template<typename RhsT, int kCpl>
__device__ __forceinline__ void fma_row(float (&acc)[kCpl], float x, const RhsT *w) {
    if constexpr (sizeof(RhsT) == 2) {
        static_assert(kCpl == 8, "fp16 rows are read 16 B per lane");
        const uint4 raw = *reinterpret_cast<const uint4 *>(w);
        const unsigned words[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            acc[2 * k] = __builtin_fmaf(x, h2f(static_cast<std::uint16_t>(words[k] & 0xffffu)),
                                        acc[2 * k]);
            acc[2 * k + 1] = __builtin_fmaf(x, h2f(static_cast<std::uint16_t>(words[k] >> 16)),
                                            acc[2 * k + 1]);
        }
    } else {
        static_assert(kCpl == 4, "fp32 rows are read 16 B per lane");
        const float4 v = *reinterpret_cast<const float4 *>(w);
        acc[0] = __builtin_fmaf(x, v.x, acc[0]);
        acc[1] = __builtin_fmaf(x, v.y, acc[1]);
        acc[2] = __builtin_fmaf(x, v.z, acc[2]);
        acc[3] = __builtin_fmaf(x, v.w, acc[3]);
    }
}

// Shape constants of the row-wave fast path: kCpl output columns per lane (16 B of W),
// kLpe lanes per entry, kEps entries per step.
template<typename RhsT, int kN>
struct WaveShape {
    static constexpr int kCpl = 16 / static_cast<int>(sizeof(RhsT));
    static constexpr int kLpe = kN / kCpl;
    static constexpr int kEps = kWave / kLpe;
    static_assert(kN % kCpl == 0 && kLpe <= kWave && kWave % kLpe == 0, "bad shape");
};

// Accumulates entries [sb, se) of row `row` (whose entries start at nnz offset `begin`)
// into this lane's kCpl partial output columns; `stage` is the wave's 64 staging slots.
template<int kBits, int kPolicy, ValueMode kMode, typename RhsT, int kN>
__device__ __forceinline__ void accumulate_segment(const QcsrArgs &a, int2 *stage, std::uint32_t row,
                                                   std::int64_t begin, std::int64_t sb,
                                                   std::int64_t se, int lane,
                                                   float (&acc)[WaveShape<RhsT, kN>::kCpl]) {
    using S = WaveShape<RhsT, kN>;
    constexpr int kCpl = S::kCpl, kLpe = S::kLpe, kEps = S::kEps;
    const int g = lane / kLpe;
    const int j = lane % kLpe;
    const std::uint8_t *pbase = nullptr;
    float row_offset = 0.0f;
    if constexpr (kMode == ValueMode::quantized) {
        pbase = a.packed + a.packed_row_ptr[row];
        if constexpr (kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
            row_offset = a.row_offsets != nullptr ? a.row_offsets[row] : 0.0f;
    }
    const RhsT *rhs = static_cast<const RhsT *>(a.rhs) + j * kCpl;
    for (std::int64_t c0 = sb; c0 < se; c0 += kWave) {
        const std::int64_t i = c0 + lane;
        int col = 0;
        float x = 0.0f;
        if (i < se) x = load_entry<kBits, kPolicy, kMode>(a, i, begin, pbase, row_offset, col);
        stage[lane] = make_int2(col, __float_as_int(x));
        wave_sync();
        const int count = se - c0 < kWave ? static_cast<int>(se - c0) : kWave;
        if (count == kWave) {
#pragma unroll
            for (int s = 0; s < kWave; s += kEps) {
                const int2 e = stage[s + g];
                fma_row<RhsT, kCpl>(acc, __int_as_float(e.y),
                                    rhs + static_cast<std::int64_t>(e.x) * a.rhs_ld);
            }
        } else {
            for (int s = 0; s < count; s += kEps) {
                if (s + g < count) {
                    const int2 e = stage[s + g];
                    fma_row<RhsT, kCpl>(acc, __int_as_float(e.y),
                                        rhs + static_cast<std::int64_t>(e.x) * a.rhs_ld);
                }
            }
        }
        wave_sync();
    }
}

// Sums the kEps group partials: lanes of equal j differ in the bits above log2(kLpe).
template<int kLpe, int kCpl>
__device__ __forceinline__ void reduce_groups(float (&acc)[kCpl]) {
    constexpr int kFirstBit = __builtin_ctz(kLpe);
#pragma unroll
    for (int k = 0; k < kCpl; ++k) {
        if constexpr (kFirstBit < 6) acc[k] = xor_reduce<kFirstBit, 5>(acc[k]);
    }
}

// Group-0 lane j: columns [j kCpl, j kCpl + kCpl) of row `row`, through the epilogue.
template<int kCpl>
__device__ __forceinline__ void store_row(const QcsrArgs &a, std::uint32_t row, int j,
                                          float (&acc)[kCpl]) {
    float *dst = a.out + static_cast<std::int64_t>(row) * a.out_ld + j * kCpl;
    if (a.ep.active) {
#pragma unroll
        for (int k = 0; k < kCpl; ++k) acc[k] = epilogue_value(a.ep, acc[k], row, j * kCpl + k);
    }
#pragma unroll
    for (int k = 0; k < kCpl; k += 4)
        *reinterpret_cast<float4 *>(dst + k) = make_float4(acc[k], acc[k + 1], acc[k + 2], acc[k + 3]);
}

template<int kBits, int kPolicy, ValueMode kMode, typename RhsT, int kN>
__global__ __launch_bounds__(kWave *kWavesPerBlock) void qcsr_spmm_rowwave(QcsrArgs a) {
    using S = WaveShape<RhsT, kN>;
    __shared__ int2 stage[kWavesPerBlock][kWave];
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t row = blockIdx.x * kWavesPerBlock + wave;
    if (row >= a.rows) return;
    const std::int64_t begin = a.row_ptr[row];
    const std::int64_t end = a.row_ptr[row + 1];
    float acc[S::kCpl];
#pragma unroll
    for (int k = 0; k < S::kCpl; ++k) acc[k] = 0.0f;
    accumulate_segment<kBits, kPolicy, kMode, RhsT, kN>(a, stage[wave], row, begin, begin, end, lane, acc);
    reduce_groups<S::kLpe, S::kCpl>(acc);
    if (lane < S::kLpe) store_row<S::kCpl>(a, row, lane, acc);
}

// ---- load-balanced form: equal nnz chunks, one wave per chunk ----------------------------

struct Balance {
    std::int64_t nnz;
    float *partials;       // [chunks][2][kN]: slot 0 = row begun before the chunk, 1 = row
                           // continuing past it
    std::uint32_t chunk;   // entries per chunk
    std::uint32_t chunks;
};

// First row a chunk starting at entry `cb` visits: the row holding entry cb, or the first
// of the (possibly empty) rows that start at cb.
__device__ __forceinline__ std::uint32_t first_row_of_chunk(const std::int32_t *row_ptr,
                                                            std::uint32_t rows, std::int64_t cb) {
    std::uint32_t lo = 0u, hi = rows;  // first r with row_ptr[r] >= cb
    while (lo < hi) {
        const std::uint32_t mid = lo + (hi - lo) / 2u;
        if (row_ptr[mid] < cb) lo = mid + 1u;
        else hi = mid;
    }
    if (lo == rows || row_ptr[lo] > cb) --lo;
    return lo;
}

// Chunk k covers entries [k chunk, (k + 1) chunk) (the last one also the empty rows at the
// end). Rows wholly inside the chunk are stored (through the epilogue); the parts of rows
// that cross a chunk edge go to the chunk's partial slots for qcsr_spmm_fixup.
template<int kBits, int kPolicy, ValueMode kMode, typename RhsT, int kN>
__global__ __launch_bounds__(kWave *kWavesPerBlock) void qcsr_spmm_balanced(QcsrArgs a, Balance b) {
    using S = WaveShape<RhsT, kN>;
    __shared__ int2 stage[kWavesPerBlock][kWave];
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t k = blockIdx.x * kWavesPerBlock + wave;
    if (k >= b.chunks) return;
    const bool last = k + 1u == b.chunks;
    const std::int64_t cb = static_cast<std::int64_t>(k) * b.chunk;
    const std::int64_t ce = last ? b.nnz : cb + b.chunk;
    for (std::uint32_t r = first_row_of_chunk(a.row_ptr, a.rows, cb); r < a.rows; ++r) {
        const std::int64_t rb = a.row_ptr[r], re = a.row_ptr[r + 1];
        if (!last && rb >= ce) break;
        float acc[S::kCpl];
#pragma unroll
        for (int c = 0; c < S::kCpl; ++c) acc[c] = 0.0f;
        accumulate_segment<kBits, kPolicy, kMode, RhsT, kN>(a, stage[wave], r, rb, rb > cb ? rb : cb,
                                                            re < ce ? re : ce, lane, acc);
        reduce_groups<S::kLpe, S::kCpl>(acc);
        if (lane < S::kLpe) {
            if (rb >= cb && re <= ce) {
                store_row<S::kCpl>(a, r, lane, acc);
            } else {
                float *dst = b.partials + (static_cast<std::int64_t>(k) * 2 + (rb < cb ? 0 : 1)) * kN
                    + lane * S::kCpl;
#pragma unroll
                for (int c = 0; c < S::kCpl; c += 4)
                    *reinterpret_cast<float4 *>(dst + c) = make_float4(acc[c], acc[c + 1], acc[c + 2], acc[c + 3]);
            }
        }
    }
}

// One wave per chunk k: if the row holding k's first entry began in an earlier chunk and
// ends in k, sum its partials in chunk order (tail of its first chunk, then the heads of
// the following chunks up to k) and store it through the epilogue.
template<int kN>
__global__ __launch_bounds__(kWave *kWavesPerBlock) void qcsr_spmm_fixup(QcsrArgs a, Balance b) {
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t k = blockIdx.x * kWavesPerBlock + wave;
    if (k >= b.chunks) return;
    const bool last = k + 1u == b.chunks;
    const std::int64_t cb = static_cast<std::int64_t>(k) * b.chunk;
    const std::int64_t ce = last ? b.nnz : cb + b.chunk;
    const std::uint32_t r = first_row_of_chunk(a.row_ptr, a.rows, cb);
    if (r >= a.rows) return;  // row_ptr[0] != 0: nothing here is well defined
    const std::int64_t rb = a.row_ptr[r], re = a.row_ptr[r + 1];
    if (!(rb < cb && re <= ce)) return;
    const std::uint32_t k0 = static_cast<std::uint32_t>(rb / b.chunk);
    for (int c = lane; c < kN; c += kWave) {
        float v = b.partials[(static_cast<std::int64_t>(k0) * 2 + 1) * kN + c];
        for (std::uint32_t q = k0 + 1u; q <= k; ++q) v += b.partials[static_cast<std::int64_t>(q) * 2 * kN + c];
        a.out[static_cast<std::int64_t>(r) * a.out_ld + c] = a.ep.active ? epilogue_value(a.ep, v, r, c) : v;
    }
}

// Generic shape: one wave per row, lanes over output columns in chunks of 64, entries
// consumed in nnz order (wave-uniform decode).
template<int kBits, int kPolicy, ValueMode kMode, typename RhsT>
__global__ __launch_bounds__(kWave *kWavesPerBlock) void qcsr_spmm_generic(QcsrArgs a,
                                                                           std::int64_t n) {
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t row = blockIdx.x * kWavesPerBlock + wave;
    if (row >= a.rows) return;
    const std::int64_t begin = a.row_ptr[row];
    const std::int64_t end = a.row_ptr[row + 1];
    const std::uint8_t *pbase = nullptr;
    float row_offset = 0.0f;
    if constexpr (kMode == ValueMode::quantized) {
        pbase = a.packed + a.packed_row_ptr[row];
        if constexpr (kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
            row_offset = a.row_offsets != nullptr ? a.row_offsets[row] : 0.0f;
    }
    const RhsT *rhs = static_cast<const RhsT *>(a.rhs);
    for (std::int64_t c0 = 0; c0 < n; c0 += kWave) {
        const std::int64_t c = c0 + lane;
        float acc = 0.0f;
        for (std::int64_t i = begin; i < end; ++i) {
            int col = 0;
            const float x = load_entry<kBits, kPolicy, kMode>(a, i, begin, pbase, row_offset, col);
            if (c < n) {
                const RhsT w = rhs[static_cast<std::int64_t>(col) * a.rhs_ld + c];
                float wf;
                if constexpr (sizeof(RhsT) == 2) wf = h2f(w);
                else wf = w;
                acc = __builtin_fmaf(x, wf, acc);
            }
        }
        if (c < n)
            a.out[static_cast<std::int64_t>(row) * a.out_ld + c] =
                a.ep.active ? epilogue_value(a.ep, acc, row, c) : acc;
    }
}

template<int kBits, int kPolicy, ValueMode kMode, typename RhsT, int kN>
int launch_balanced(const QcsrArgs &a, const Balance &b, hipStream_t stream) {
    const dim3 grid((b.chunks + kWavesPerBlock - 1) / kWavesPerBlock), block(kWave * kWavesPerBlock);
    hipLaunchKernelGGL((qcsr_spmm_balanced<kBits, kPolicy, kMode, RhsT, kN>), grid, block, 0, stream, a, b);
    hipLaunchKernelGGL((qcsr_spmm_fixup<kN>), grid, block, 0, stream, a, b);
    return check_launch("qcsr_spmm_balanced");
}

template<int kBits, int kPolicy, ValueMode kMode, typename RhsT>
int launch_rhs(const QcsrArgs &a, std::int64_t n, bool aligned, const Balance *bal,
               hipStream_t stream) {
    const unsigned blocks = (a.rows + kWavesPerBlock - 1) / kWavesPerBlock;
    const dim3 grid(blocks), block(kWave * kWavesPerBlock);
    constexpr int kCpl = 16 / static_cast<int>(sizeof(RhsT));
    if (bal != nullptr && aligned && n == 64)
        return launch_balanced<kBits, kPolicy, kMode, RhsT, 64>(a, *bal, stream);
    if (bal != nullptr && aligned && n == 128)
        return launch_balanced<kBits, kPolicy, kMode, RhsT, 128>(a, *bal, stream);
    if (aligned && n == 64) {
        hipLaunchKernelGGL((qcsr_spmm_rowwave<kBits, kPolicy, kMode, RhsT, 64>), grid, block, 0,
                           stream, a);
    } else if (aligned && n == 128) {
        hipLaunchKernelGGL((qcsr_spmm_rowwave<kBits, kPolicy, kMode, RhsT, 128>), grid, block, 0,
                           stream, a);
    } else if (aligned && n == 32 && kCpl == 8) {
        hipLaunchKernelGGL((qcsr_spmm_rowwave<kBits, kPolicy, kMode, RhsT, 32>), grid, block, 0,
                           stream, a);
    } else {
        hipLaunchKernelGGL((qcsr_spmm_generic<kBits, kPolicy, kMode, RhsT>), grid, block, 0,
                           stream, a, n);
    }
    return check_launch("qcsr_spmm");
}

template<int kBits, int kPolicy, ValueMode kMode>
int launch_mode(const QcsrArgs &a, std::uint32_t rhs_dtype, std::int64_t n, bool aligned,
                const Balance *bal, hipStream_t stream) {
    if (rhs_dtype == CELLERATOR_DTYPE_F16)
        return launch_rhs<kBits, kPolicy, kMode, std::uint16_t>(a, n, aligned, bal, stream);
    return launch_rhs<kBits, kPolicy, kMode, float>(a, n, aligned, bal, stream);
}

template<int kPolicy>
int launch_bits(const QcsrArgs &a, std::uint32_t bits, std::uint32_t rhs_dtype, std::int64_t n,
                bool aligned, const Balance *bal, hipStream_t stream) {
    switch (bits) {
    case 1: return launch_mode<1, kPolicy, ValueMode::quantized>(a, rhs_dtype, n, aligned, bal, stream);
    case 2: return launch_mode<2, kPolicy, ValueMode::quantized>(a, rhs_dtype, n, aligned, bal, stream);
    case 4: return launch_mode<4, kPolicy, ValueMode::quantized>(a, rhs_dtype, n, aligned, bal, stream);
    case 8: return launch_mode<8, kPolicy, ValueMode::quantized>(a, rhs_dtype, n, aligned, bal, stream);
    default: return fail(CX_STATUS_UNSUPPORTED, "quantized CSR bits must be 1, 2, 4 or 8");
    }
}

__global__ void pack_gene_affine_kernel(const float *scales, const float *offsets, std::uint32_t cols,
                                        float2 *pairs) {
    const std::uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= cols) return;
    pairs[c] = make_float2(scales != nullptr ? scales[c] : 1.0f, offsets != nullptr ? offsets[c] : 0.0f);
}

bool aligned16(const void *p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0u; }

// Entries per chunk of the balanced form: about 65,536 chunks, at least 1,024 entries each,
// a multiple of 64.
std::uint32_t balance_chunk(std::uint64_t nnz) {
    std::uint64_t c = (nnz + 65535u) / 65536u;
    c = (c + 63u) / 64u * 64u;
    return static_cast<std::uint32_t>(c < 1024u ? 1024u : c);
}

std::uint64_t balance_bytes(std::uint64_t nnz, std::int64_t out_cols) {
    if (nnz == 0u || out_cols <= 0) return 0u;
    const std::uint64_t chunk = balance_chunk(nnz);
    return (nnz + chunk - 1u) / chunk * 2u * static_cast<std::uint64_t>(out_cols) * 4u;
}

// Shared body of the forward entries; `bal_ws` (may be NULL) selects the balanced form.
int qcsr_forward(const cx_qcsr_matrix *m, const void *rhs, std::uint32_t rhs_dtype, std::int64_t rhs_ld,
                 std::int64_t out_cols, float *out, std::int64_t out_ld, const cx_spmm_epilogue *epilogue,
                 void *bal_ws, std::uint64_t bal_bytes, void *stream);

} // namespace
} // namespace cx

extern "C" int cx_qcsr_spmm_fwd(const cx_qcsr_matrix *m, const void *rhs, uint32_t rhs_dtype,
                                int64_t rhs_ld, int64_t out_cols, float *out, int64_t out_ld,
                                void *stream) {
    return cx_qcsr_spmm_fwd_epilogue(m, rhs, rhs_dtype, rhs_ld, out_cols, out, out_ld, nullptr,
                                     stream);
}

extern "C" int cx_qcsr_spmm_fwd_epilogue(const cx_qcsr_matrix *m, const void *rhs,
                                         uint32_t rhs_dtype, int64_t rhs_ld, int64_t out_cols,
                                         float *out, int64_t out_ld,
                                         const cx_spmm_epilogue *epilogue, void *stream) {
    cx::clear_error();
    return cx::qcsr_forward(m, rhs, rhs_dtype, rhs_ld, out_cols, out, out_ld, epilogue, nullptr, 0u,
                            stream);
}

extern "C" int cx_qcsr_spmm_balanced_workspace(const cx_qcsr_matrix *m, int64_t out_cols,
                                               uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (m == nullptr || bytes == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_balanced_workspace: null argument");
    *bytes = balance_bytes(m->nnz, out_cols);
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_spmm_fwd_balanced(const cx_qcsr_matrix *m, const void *rhs,
                                         uint32_t rhs_dtype, int64_t rhs_ld, int64_t out_cols,
                                         float *out, int64_t out_ld,
                                         const cx_spmm_epilogue *epilogue, void *workspace,
                                         uint64_t workspace_bytes, void *stream) {
    cx::clear_error();
    return cx::qcsr_forward(m, rhs, rhs_dtype, rhs_ld, out_cols, out, out_ld, epilogue, workspace,
                            workspace_bytes, stream);
}

namespace cx {
namespace {

int qcsr_forward(const cx_qcsr_matrix *m, const void *rhs, std::uint32_t rhs_dtype, std::int64_t rhs_ld,
                 std::int64_t out_cols, float *out, std::int64_t out_ld, const cx_spmm_epilogue *epilogue,
                 void *bal_ws, std::uint64_t bal_bytes, void *stream) {
    if (m == nullptr || out == nullptr || rhs == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd: null matrix, rhs or output");
    if (rhs_dtype != CELLERATOR_DTYPE_F16 && rhs_dtype != CELLERATOR_DTYPE_F32)
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_spmm_fwd: rhs dtype must be F16 or F32");
    if (out_cols <= 0 || rhs_ld < out_cols || out_ld < out_cols)
        return fail(CX_STATUS_INVALID_SHAPE,
                    "cx_qcsr_spmm_fwd: out_cols must be positive and <= both leading dimensions");
    if (m->rows == 0u) return CX_STATUS_SUCCESS;
    if (m->row_ptr == nullptr || (m->nnz != 0u && m->col_idx == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd: null row_ptr or col_idx");
    if (m->nnz > static_cast<std::uint64_t>(INT32_MAX))
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_fwd: nnz exceeds int32 row offsets");
    if (m->bits != 0u) {
        if (m->packed_row_ptr == nullptr || (m->nnz != 0u && m->packed_values == nullptr))
            return fail(CX_STATUS_INVALID_ARGUMENT,
                        "cx_qcsr_spmm_fwd: quantized matrix needs packed_row_ptr and packed_values");
        if (m->decode_policy != CX_DECODE_PER_GENE_AFFINE
            && m->decode_policy != CX_DECODE_COLUMN_SCALE_ROW_OFFSET
            && m->decode_policy != CX_DECODE_PER_GENE_AFFINE_PAIRS)
            return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_spmm_fwd: unknown decode policy");
        if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS
            && (m->column_scales == nullptr || m->column_offsets != nullptr
                || (reinterpret_cast<std::uintptr_t>(m->column_scales) & 7u) != 0u))
            return fail(CX_STATUS_INVALID_ARGUMENT,
                        "cx_qcsr_spmm_fwd: interleaved metadata needs 8-byte aligned (scale, offset) "
                        "pairs in column_scales and NULL column_offsets");
    } else {
        if (m->nnz != 0u && m->values == nullptr)
            return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd: null values");
        if (m->value_dtype != CELLERATOR_DTYPE_F16 && m->value_dtype != CELLERATOR_DTYPE_F32)
            return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_spmm_fwd: value dtype must be F16 or F32");
    }
    if (static_cast<const void *>(out) == rhs)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd: output aliases the rhs");
    Epilogue ep;
    const int erc = make_epilogue(epilogue, m->rows, out_cols, out, out_ld, &ep, "cx_qcsr_spmm_fwd");
    if (erc != CX_STATUS_SUCCESS) return erc;

    QcsrArgs a{};
    a.ep = ep;
    a.row_ptr = m->row_ptr;
    a.packed_row_ptr = m->packed_row_ptr;
    a.col_idx = m->col_idx;
    a.packed = m->packed_values;
    a.scales = m->column_scales;
    a.offsets = m->column_offsets;
    a.row_offsets = m->row_offsets;
    a.values = m->values;
    a.rhs = rhs;
    a.rhs_ld = rhs_ld;
    a.out = out;
    a.out_ld = out_ld;
    a.rows = m->rows;
    a.cols = m->cols;
    a.flags = m->flags;
    const std::size_t esize = rhs_dtype == CELLERATOR_DTYPE_F16 ? 2u : 4u;
    const bool aligned = aligned16(rhs) && aligned16(out) && (rhs_ld * esize) % 16 == 0
        && (out_ld * 4) % 16 == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    Balance balance{};
    const Balance *bal = nullptr;
    if (bal_ws != nullptr && m->nnz != 0u) {
        if (bal_bytes < balance_bytes(m->nnz, out_cols))
            return fail(CX_STATUS_INVALID_ARGUMENT,
                        "cx_qcsr_spmm_fwd_balanced: workspace smaller than cx_qcsr_spmm_balanced_workspace");
        if ((reinterpret_cast<std::uintptr_t>(bal_ws) & 15u) != 0u)
            return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_balanced: workspace must be 16-byte aligned");
        balance.nnz = static_cast<std::int64_t>(m->nnz);
        balance.partials = static_cast<float *>(bal_ws);
        balance.chunk = balance_chunk(m->nnz);
        balance.chunks = static_cast<std::uint32_t>((m->nnz + balance.chunk - 1u) / balance.chunk);
        bal = &balance;
    }
    if (bal == nullptr && qcsr_parts_applicable(a, m->bits, rhs_dtype, out_cols, aligned))
        return launch_qcsr_parts(a, m->bits, m->decode_policy, out_cols, s);
    if (m->bits == 0u) {
        if (m->value_dtype == CELLERATOR_DTYPE_F16)
            return launch_mode<0, CX_DECODE_PER_GENE_AFFINE, ValueMode::f16>(a, rhs_dtype,
                                                                               out_cols, aligned, bal, s);
        return launch_mode<0, CX_DECODE_PER_GENE_AFFINE, ValueMode::f32>(a, rhs_dtype, out_cols,
                                                                          aligned, bal, s);
    }
    if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE)
        return launch_bits<CX_DECODE_PER_GENE_AFFINE>(a, m->bits, rhs_dtype, out_cols, aligned, bal, s);
    if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS)
        return launch_bits<CX_DECODE_PER_GENE_AFFINE_PAIRS>(a, m->bits, rhs_dtype, out_cols, aligned, bal, s);
    return launch_bits<CX_DECODE_COLUMN_SCALE_ROW_OFFSET>(a, m->bits, rhs_dtype, out_cols, aligned,
                                                          bal, s);
}

} // namespace
} // namespace cx

namespace cx {
namespace {

__global__ void check_columns_init(std::uint32_t *flag) { *flag = CX_QCSR_COLUMNS_SORTED; }

// One wave per row (grid-stride): any column outside [0, cols) or above its successor in the
// row clears the flag.
__global__ __launch_bounds__(256) void check_columns_kernel(const std::int32_t *row_ptr, const std::int32_t *col_idx,
                                                            std::uint32_t rows, std::int32_t cols, std::uint32_t *flag) {
    const std::uint32_t lane = threadIdx.x % kWave;
    const std::uint32_t waves = gridDim.x * (blockDim.x / kWave);
    bool bad = false;
    for (std::uint32_t r = (blockIdx.x * blockDim.x + threadIdx.x) / kWave; r < rows; r += waves) {
        const std::int32_t b = row_ptr[r], e = row_ptr[r + 1];
        for (std::int32_t i = b + static_cast<std::int32_t>(lane); i < e; i += kWave) {
            const std::int32_t c = col_idx[i];
            bad = bad || c < 0 || c >= cols || (i + 1 < e && c > col_idx[i + 1]);
        }
    }
    if (__ballot(bad) != 0ull && lane == 0u) atomicAnd(flag, 0u);
}

} // namespace
} // namespace cx

extern "C" int cx_qcsr_check_columns(const cx_qcsr_matrix *m, uint32_t *device_flag, void *stream) {
    using namespace cx;
    clear_error();
    if (m == nullptr || device_flag == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_check_columns: null matrix or flag");
    if (m->rows != 0u && (m->row_ptr == nullptr || (m->nnz != 0u && m->col_idx == nullptr)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_check_columns: missing row_ptr or col_idx");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(check_columns_init, dim3(1), dim3(1), 0, s, device_flag);
    if (m->rows != 0u) {
        const std::uint32_t blocks = std::min<std::uint32_t>((m->rows + 3u) / 4u, 8192u);
        hipLaunchKernelGGL(check_columns_kernel, dim3(blocks), dim3(256), 0, s, m->row_ptr, m->col_idx, m->rows,
                           static_cast<std::int32_t>(std::min<std::uint32_t>(m->cols, INT32_MAX)), device_flag);
    }
    return check_launch("cx_qcsr_check_columns");
}

extern "C" int cx_qcsr_check_columns_sync(const cx_qcsr_matrix *m, uint32_t *host_flag, void *stream) {
    using namespace cx;
    clear_error();
    if (host_flag == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_check_columns_sync: null flag");
    *host_flag = 0u;
    std::uint32_t *flag = nullptr;
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&flag), sizeof(std::uint32_t));
    if (e != hipSuccess) return hip_fail(e, "cx_qcsr_check_columns_sync: hipMalloc");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = cx_qcsr_check_columns(m, flag, stream);
    if (rc == CX_STATUS_SUCCESS) {
        e = hipMemcpyAsync(host_flag, flag, sizeof(std::uint32_t), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "cx_qcsr_check_columns_sync");
    }
    (void)hipFree(flag);
    return rc;
}

extern "C" int cx_stream_synchronize(void *stream) {
    cx::clear_error();
    const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    return e == hipSuccess ? CX_STATUS_SUCCESS : cx::hip_fail(e, "cx_stream_synchronize");
}

extern "C" int cx_qcsr_pack_gene_affine(const float *scales, const float *offsets, uint32_t cols,
                                        float *pairs, void *stream) {
    using namespace cx;
    clear_error();
    if (pairs == nullptr || (reinterpret_cast<std::uintptr_t>(pairs) & 7u) != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_pack_gene_affine: pairs must be 8-byte aligned");
    if (pairs == scales || pairs == offsets)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_pack_gene_affine: pairs aliases an input");
    if (cols == 0u) return CX_STATUS_SUCCESS;
    hipLaunchKernelGGL(pack_gene_affine_kernel, dim3((cols + 255u) / 256u), dim3(256), 0,
                       static_cast<hipStream_t>(stream), scales, offsets, cols,
                       reinterpret_cast<float2 *>(pairs));
    return check_launch("cx_qcsr_pack_gene_affine");
}

// ---- allocation-free balanced forward -------------------------------------------------------
//
// The balanced form's only scratch is the partial rows of the rows that cross a chunk edge:
// at most 65,536 chunks x 2 slots x N fp32. This entry keeps them in a device array of this
// library (one per GPU, held until the process ends) instead of a caller workspace, so
// callers that cannot allocate (graph capture, tight serving loops) can still run it. Every
// slot the fixup reads is written by the same launch first, so the array is never cleared.
// Calls that overlap on one GPU share the array and race.

namespace {
constexpr std::uint64_t kNoAllocScratchBytes = 32ull << 20;  // 65,536 chunks x 2 x 64 fp32
constexpr int kNoAllocMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_noalloc_lock;
void *g_noalloc_ptr[kNoAllocMaxDevices] = {};

// Device address of `scratch` on the stream's device, resolved once per device with that
// device current (the host-side name is only a stand-in for the symbol).
int noalloc_scratch(hipStream_t stream, void **out) {
    int current = 0;
    hipError_t e = hipGetDevice(&current);
    if (e != hipSuccess) return cx::hip_fail(e, "cx_qcsr_spmm_fwd_balanced_noalloc: hipGetDevice");
    int device = current;
    if (stream != nullptr) {
        e = hipStreamGetDevice(stream, &device);
        if (e != hipSuccess) return cx::hip_fail(e, "cx_qcsr_spmm_fwd_balanced_noalloc: hipStreamGetDevice");
    }
    if (device != current)
        return cx::fail(CX_STATUS_INVALID_ARGUMENT,
                        "cx_qcsr_spmm_fwd_balanced_noalloc: the stream's device must be the current device");
    if (device < 0 || device >= kNoAllocMaxDevices)
        return cx::fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_spmm_fwd_balanced_noalloc: device ordinal above 63");
    std::lock_guard<std::mutex> lock(g_noalloc_lock);
    if (g_noalloc_ptr[device] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return cx::hip_fail(e, "cx_qcsr_spmm_fwd_balanced_noalloc: hipGetSymbolAddress");
        g_noalloc_ptr[device] = p;
    }
    *out = g_noalloc_ptr[device];
    return CX_STATUS_SUCCESS;
}
}  // namespace

extern "C" int cx_qcsr_spmm_fwd_balanced_noalloc(const cx_qcsr_matrix *m, const void *rhs,
                                                 uint32_t rhs_dtype, int64_t rhs_ld, int64_t out_cols,
                                                 float *out, int64_t out_ld,
                                                 const cx_spmm_epilogue *epilogue, void *stream) {
    cx::clear_error();
    if (m == nullptr)
        return cx::fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_balanced_noalloc: null matrix");
    // only the 64- and 128-column balanced kernels use partial rows
    const std::uint64_t need = out_cols == 64 || out_cols == 128 ? cx::balance_bytes(m->nnz, out_cols) : 0u;
    if (need > kNoAllocScratchBytes) {
        cx::set_error("cx_qcsr_spmm_fwd_balanced_noalloc: %llu bytes of partial rows exceed the %llu-byte "
                      "scratch (use cx_qcsr_spmm_fwd_balanced with a workspace)",
                      static_cast<unsigned long long>(need),
                      static_cast<unsigned long long>(kNoAllocScratchBytes));
        return CX_STATUS_INVALID_SHAPE;
    }
    void *ws = nullptr;
    const int rc = noalloc_scratch(static_cast<hipStream_t>(stream), &ws);
    if (rc != CX_STATUS_SUCCESS) return rc;
    return cx::qcsr_forward(m, rhs, rhs_dtype, rhs_ld, out_cols, out, out_ld, epilogue, ws,
                            kNoAllocScratchBytes, stream);
}
