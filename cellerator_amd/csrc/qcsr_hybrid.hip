// qcsr_hybrid.hip -- quantized CSR SpMM in execution order with a dense head on the matrix
// cores (fp16 weights, 64 output columns per launch).
//
// In an execution order that puts the most frequently stored genes first (the popularity
// order of exec_order.hip, or any frozen plan order), the first H genes of a single-cell
// matrix are stored in a large share of the cells: at C3, the first 4,096 of 33,538 genes
// hold 2/3 of the nonzeros at 24% mean density (93% for the first 256). Those columns are
// dense enough for the matrix cores. The head kernel here computes Y_head = X[:, 0:H) .
// W[0:H, :] with v_mfma_f32_16x16x32_f16; the tail X[:, H:) . W[H:, :] runs on the row-group
// VALU kernel of qcsr_parts.hip, which starts every row at its first entry >= H (recorded
// here) and adds Y_head before its epilogue.
//
// Exactness. Each stored code is decoded exactly as the reference codec does,
// x = fma(float(code), scale, offset) in fp32 (include/Cellerator/quantized/access.cuh:81-91),
// and then split into three fp16 parts x = hi + mid + lo (each the round-to-nearest fp16 of
// the remaining residual; the residuals are exact in fp32). For |x| in [2^-2, 2^15) the
// three parts hold all 24 bits of x, so hi + mid + lo == x exactly; below 2^-2 the lowest
// part may lose bits under 2^-24 (an absolute error below 2^-25 |w|). Each part times an
// fp16 weight (11 x 11 bits) is exact in fp32, and the matrix cores accumulate in fp32: the
// result differs from an fp32 FMA chain only in summation order. The host rejects head
// genes whose decoded values can reach 2^15.
//
// Layout per workgroup (8 waves, 256 rows): the genes of the head are walked in slabs of 64
// (two 32-gene MFMA chunks). Per slab:
//   * the slab's packed weights ([chunk][column][32 genes], 8 KB) and per-gene metadata are
//     double-buffered in LDS, loaded one slab ahead into registers by all waves;
//   * each wave owns 32 rows (two 16-row MFMA blocks) and an LDS tile of 3 planes (hi, mid,
//     lo) x 32 rows x 64 genes of fp16, zeroed, then filled with the decoded entries of its
//     rows that fall in the slab (2 lanes per row, 4 consecutive entries per lane per step,
//     the row's cursor advanced by the run it found);
//   * per chunk: 4 weight fragments (one per 16-column tile of the 64 outputs) and per row
//     block 3 value fragments, 24 MFMAs into 2 x 4 fp32 accumulator tiles.
// Operands: A = W^T (output column x gene), B = X^T (gene x cell row), so each lane ends with
// 4 consecutive output columns of one row (a 16-byte store).
#include "qcsr_common.hpp"

#include <algorithm>
#include <cstring>

typedef _Float16 cx_half8 __attribute__((ext_vector_type(8)));
typedef float cx_float4 __attribute__((ext_vector_type(4)));

namespace cx {
namespace {

constexpr int kHeadWaves = 8;
constexpr int kRowsPerWave = 32;
constexpr int kHeadRows = kHeadWaves * kRowsPerWave;  // rows per workgroup
constexpr int kSlab = 64;                              // genes per slab
constexpr int kXStride = kSlab + 8;                    // fp16 per tile row (16 B pad: the 16 rows of a fragment read fall in distinct banks)
constexpr int kWStride = 40;                           // fp16 per panel column in LDS (32 genes + 16 B pad)

struct HeadShared {
    _Float16 x[kHeadWaves][3][kRowsPerWave][kXStride];
    _Float16 w[2][2][64][kWStride];
    float2 meta[2][kSlab];
};

struct HeadArgs {
    const std::int32_t *row_ptr;
    const std::int32_t *packed_row_ptr;
    const std::int32_t *col_idx;
    const std::uint8_t *packed;
    const float *scales;   // per gene, or (scale, offset) pairs for the pairs policy
    const float *offsets;
    const float *row_offsets;
    const std::uint16_t *panel;  // fp16 [head/32][panel_n][32] at this launch's first column
    float *partial;              // [rows][64] fp32: Y_head
    std::int32_t *head_end;      // [rows]: first entry of each row with gene >= head
    std::uint32_t rows;
    std::uint32_t head;          // head genes, a multiple of kSlab
    std::uint32_t panel_n;       // output columns of the packed panel
};

__device__ __forceinline__ uint4 ldg4(const void *p) { return *static_cast<const uint4 *>(p); }

template<int kPolicy>
__device__ __forceinline__ float2 gene_meta(const HeadArgs &h, std::uint32_t g) {
    if constexpr (kPolicy == CX_DECODE_PER_GENE_AFFINE_PAIRS) {
        return reinterpret_cast<const float2 *>(h.scales)[g];
    } else {
        const float s = h.scales != nullptr ? h.scales[g] : 1.0f;
        const float o = kPolicy == CX_DECODE_PER_GENE_AFFINE && h.offsets != nullptr ? h.offsets[g] : 0.0f;
        return make_float2(s, o);
    }
}

template<int kBits, int kPolicy>
__global__ __launch_bounds__(kHeadWaves * kWave) void qcsr_head_mfma(HeadArgs h) {
    __shared__ HeadShared sh;
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const std::uint32_t wave_first = blockIdx.x * static_cast<std::uint32_t>(kHeadRows) + wave * kRowsPerWave;

    // ---- scatter role: lanes 2r, 2r + 1 walk row r of the wave -------------------------
    const int rr = lane >> 1;
    const int sub = lane & 1;
    const std::uint32_t row = wave_first + static_cast<std::uint32_t>(rr);
    const bool has_row = row < h.rows;
    std::int32_t cur = 0, end = 0, rbeg = 0;
    std::int64_t pbyte = 0;
    float roff = 0.0f;
    if (has_row) {
        rbeg = cur = h.row_ptr[row];
        end = h.row_ptr[row + 1];
        pbyte = h.packed_row_ptr[row];
        if constexpr (kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
            roff = h.row_offsets != nullptr ? h.row_offsets[row] : 0.0f;
    }

    // ---- weight slab staging: thread tid moves one 16-byte piece of the slab's panel -----
    const int wc = tid >> 8;            // chunk of the slab
    const int wcol = (tid >> 2) & 63;   // output column
    const int wpiece = tid & 3;         // 8 genes
    // bounds of the entry and code arrays: the matrix's own extent
    const std::int64_t nnz_all = h.row_ptr[h.rows];
    const std::int64_t packed_bytes = h.packed_row_ptr[h.rows];
    auto load_slab = [&](std::uint32_t s, uint4 &wv, float2 &mv) {
        const std::uint64_t chunk = 2u * s + static_cast<std::uint32_t>(wc);
        wv = ldg4(h.panel + ((chunk * h.panel_n + static_cast<std::uint32_t>(wcol)) * 32u + wpiece * 8u));
        if (tid < kSlab) mv = gene_meta<kPolicy>(h, s * kSlab + static_cast<std::uint32_t>(tid));
    };
    auto store_slab = [&](int buf, const uint4 &wv, const float2 &mv) {
        *reinterpret_cast<uint4 *>(&sh.w[buf][wc][wcol][wpiece * 8]) = wv;
        if (tid < kSlab) sh.meta[buf][tid] = mv;
    };

    // acc sums the hi and mid parts; acc_lo the lo parts, which are stored scaled by 2^12
    // (an exact power-of-two scale) so they stay normal fp16 numbers: the matrix cores are
    // not relied on to keep fp16 subnormal inputs
    cx_float4 acc[2][4], acc_lo[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[b][t] = acc_lo[b][t] = cx_float4{0.0f, 0.0f, 0.0f, 0.0f};

    const std::uint32_t slabs = h.head / kSlab;
    uint4 wnext = make_uint4(0u, 0u, 0u, 0u);
    float2 mnext = make_float2(0.0f, 0.0f);
    if (slabs != 0u) {
        load_slab(0u, wnext, mnext);
        store_slab(0, wnext, mnext);
    }
    __syncthreads();

    _Float16 *xw = &sh.x[wave][0][0][0];
    constexpr std::uint32_t kMask = (1u << kBits) - 1u;
    for (std::uint32_t s = 0; s < slabs; ++s) {
        const int buf = static_cast<int>(s & 1u);
        if (s + 1u < slabs) load_slab(s + 1u, wnext, mnext);

        // zero this wave's tiles: 3 planes x 32 rows x 64 genes (768 pieces of 16 bytes)
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            const int piece = k * kWave + lane;             // 0 .. 767
            const int plane = piece >> 8, r = (piece >> 3) & 31, c8 = piece & 7;
            *reinterpret_cast<uint4 *>(&sh.x[wave][plane][r][c8 * 8]) = make_uint4(0u, 0u, 0u, 0u);
        }

        // scatter the decoded entries of the slab: step by 8 entries per row
        const std::int32_t lo = static_cast<std::int32_t>(s * kSlab);
        const std::int32_t hi = lo + kSlab;
        const float2 *meta = sh.meta[buf];
        bool active = has_row && cur < end;
        while (__builtin_amdgcn_ballot_w64(active) != 0u) {
            int n_in = 0;
            if (active) {
                const std::int32_t e0 = cur + 4 * sub;
                std::int32_t c[4];
                if (static_cast<std::int64_t>(e0) + 4 <= nnz_all) {
                    const uint4 v = ldg4(h.col_idx + e0);
                    c[0] = static_cast<std::int32_t>(v.x); c[1] = static_cast<std::int32_t>(v.y);
                    c[2] = static_cast<std::int32_t>(v.z); c[3] = static_cast<std::int32_t>(v.w);
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) c[k] = e0 + k < nnz_all ? h.col_idx[e0 + k] : 0x7fffffff;
                }
                // codes of entries e0 .. e0 + 3: an aligned dword pair around their first bit
                const std::int64_t bit = (pbyte << 3) + static_cast<std::int64_t>(e0 - rbeg) * kBits;
                const std::int64_t al = (bit >> 3) & ~static_cast<std::int64_t>(3);
                std::uint32_t d0, d1;
                if (al + 8 <= packed_bytes) {
                    const uint2 d = *reinterpret_cast<const uint2 *>(h.packed + al);
                    d0 = d.x; d1 = d.y;
                } else {
                    d0 = d1 = 0u;
#pragma unroll
                    for (int b = 0; b < 8; ++b) {
                        const std::uint32_t v = al + b < packed_bytes ? h.packed[al + b] : 0u;
                        if (b < 4) d0 |= v << (8 * b);
                        else d1 |= v << (8 * (b - 4));
                    }
                }
                const std::uint32_t cw = __builtin_amdgcn_alignbit(d1, d0, static_cast<std::uint32_t>(bit - (al << 3)));
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    // sorted rows (the launch requires it): a run entry is in [lo, hi); the
                    // lower bound only keeps a broken promise inside the tile
                    const bool in = e0 + k < end && c[k] < hi && c[k] >= lo;
                    if (in) {
                        const int g = c[k] - lo;
                        const float2 md = meta[g];
                        const float off = kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET ? roff : md.y;
                        const float x = __builtin_fmaf(static_cast<float>((cw >> (k * kBits)) & kMask), md.x, off);
                        const _Float16 p0 = static_cast<_Float16>(x);
                        const float r1 = x - static_cast<float>(p0);
                        const _Float16 p1 = static_cast<_Float16>(r1);
                        const _Float16 p2 = static_cast<_Float16>((r1 - static_cast<float>(p1)) * 4096.0f);
                        _Float16 *px = xw + rr * kXStride + g;
                        px[0] = p0;
                        px[kRowsPerWave * kXStride] = p1;
                        px[2 * kRowsPerWave * kXStride] = p2;
                        ++n_in;
                    }
                }
            }
            // both lanes of a row advance by the entries the pair found in the slab
            const int total = n_in + __shfl_xor(n_in, 1, kWave);
            cur += total;
            active = active && total == 8 && cur < end;
        }

        // matrix cores: two 32-gene chunks
        const int fr = lane & 15;        // A row / B column / D column of this lane
        const int fk = (lane >> 4) * 8;  // first gene of this lane's fragment
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            cx_half8 aw[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                aw[t] = *reinterpret_cast<const cx_half8 *>(&sh.w[buf][c][t * 16 + fr][fk]);
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                cx_half8 bx[3];
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    bx[p] = *reinterpret_cast<const cx_half8 *>(&sh.x[wave][p][b * 16 + fr][c * 32 + fk]);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[t], bx[0], acc[b][t], 0, 0, 0);
                    acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[t], bx[1], acc[b][t], 0, 0, 0);
                    acc_lo[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[t], bx[2], acc_lo[b][t], 0, 0, 0);
                }
            }
        }

        if (s + 1u < slabs) store_slab(buf ^ 1, wnext, mnext);
        __syncthreads();
    }

    // Y_head: lane holds columns t*16 + 4*(lane/16) .. +3 of row (lane % 16) of each block
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const std::uint32_t r = wave_first + static_cast<std::uint32_t>(b * 16 + (lane & 15));
        if (r < h.rows) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = __builtin_fmaf(acc_lo[b][t][i], 1.0f / 4096.0f, acc[b][t][i]);
                float *o = h.partial + static_cast<std::int64_t>(r) * 64 + t * 16 + 4 * (lane >> 4);
                *reinterpret_cast<float4 *>(o) = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
    if (has_row && sub == 0) h.head_end[row] = cur;
}

} // namespace

// Launches the head kernel for codes of `bits` under `policy` (validated by the caller).
int launch_qcsr_head(const QcsrArgs &a, std::uint32_t bits, std::uint32_t policy, std::uint32_t head,
                     const std::uint16_t *panel, std::uint32_t panel_n, float *partial, std::int32_t *head_end,
                     hipStream_t stream) {
    HeadArgs h{};
    h.row_ptr = a.row_ptr;
    h.packed_row_ptr = a.packed_row_ptr;
    h.col_idx = a.col_idx;
    h.packed = a.packed;
    h.scales = a.scales;
    h.offsets = a.offsets;
    h.row_offsets = a.row_offsets;
    h.panel = panel;
    h.partial = partial;
    h.head_end = head_end;
    h.rows = a.rows;
    h.head = head;
    h.panel_n = panel_n;
    const dim3 grid((a.rows + kHeadRows - 1) / kHeadRows), block(kHeadWaves * kWave);
#define CX_HEAD(B, P) hipLaunchKernelGGL((qcsr_head_mfma<B, P>), grid, block, 0, stream, h)
#define CX_HEAD_POLICY(B)                                                                   \
    do {                                                                                    \
        if (policy == CX_DECODE_PER_GENE_AFFINE) CX_HEAD(B, CX_DECODE_PER_GENE_AFFINE);     \
        else if (policy == CX_DECODE_PER_GENE_AFFINE_PAIRS) CX_HEAD(B, CX_DECODE_PER_GENE_AFFINE_PAIRS); \
        else CX_HEAD(B, CX_DECODE_COLUMN_SCALE_ROW_OFFSET);                                 \
    } while (0)
    switch (bits) {
    case 1: CX_HEAD_POLICY(1); break;
    case 2: CX_HEAD_POLICY(2); break;
    case 4: CX_HEAD_POLICY(4); break;
    default: CX_HEAD_POLICY(8); break;
    }
#undef CX_HEAD_POLICY
#undef CX_HEAD
    return check_launch("qcsr_head_mfma");
}

} // namespace cx

namespace cx {
namespace {

// Largest |decoded value| any code of a head gene can take, as float bits (non-negative
// floats order like their bit patterns): per-gene affine max(|o|, |o + qmax s|); column
// scale with row offsets |s| qmax (the row offsets' largest magnitude is added by the host).
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
        if (!(b == b)) b = __builtin_huge_valf();  // NaN metadata: reject
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

__global__ void zero_two_words(std::uint32_t *p) { p[0] = 0u; p[1] = 0u; }

constexpr float kHeadValueLimit = 32768.0f;  // fp16 parts of |x| < 2^15 cannot overflow

bool valid_bits(std::uint32_t b) { return b == 1u || b == 2u || b == 4u || b == 8u; }

int validate_hybrid(const cx_qcsr_matrix *m, std::uint32_t head, const char *who) {
    if (m == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, who);
    if (!valid_bits(m->bits))
        return fail(CX_STATUS_UNSUPPORTED, "hybrid quantized CSR: codes of 1, 2, 4 or 8 bits only");
    if (m->decode_policy != CX_DECODE_PER_GENE_AFFINE && m->decode_policy != CX_DECODE_PER_GENE_AFFINE_PAIRS
        && m->decode_policy != CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
        return fail(CX_STATUS_UNSUPPORTED, "hybrid quantized CSR: unknown decode policy");
    if (head % 1024u != 0u || head > m->cols)
        return fail(CX_STATUS_INVALID_SHAPE, "hybrid quantized CSR: head_cols must be a multiple of 1,024 within cols");
    if (m->rows != 0u && (m->row_ptr == nullptr || m->packed_row_ptr == nullptr
                          || (m->nnz != 0u && (m->col_idx == nullptr || m->packed_values == nullptr))))
        return fail(CX_STATUS_INVALID_ARGUMENT, "hybrid quantized CSR: null structure or codes");
    if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS && m->column_scales == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "hybrid quantized CSR: the pairs policy needs column_scales");
    return CX_STATUS_SUCCESS;
}

} // namespace
} // namespace cx

extern "C" int cx_qcsr_hybrid_prepare(const cx_qcsr_matrix *m, uint32_t head_cols, const uint16_t *rhs_f16,
                                      int64_t rhs_ld, uint32_t out_cols, uint16_t *head_panel, void *stream) {
    using namespace cx;
    clear_error();
    int rc = validate_hybrid(m, head_cols, "cx_qcsr_hybrid_prepare: null matrix");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (head_cols == 0u) return CX_STATUS_SUCCESS;
    if (rhs_f16 == nullptr || head_panel == nullptr || out_cols == 0u || out_cols % 64u != 0u || rhs_ld < out_cols)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_hybrid_prepare: null weights or panel, or out_cols not a multiple of 64");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    std::uint32_t *words = nullptr;
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&words), 2 * sizeof(std::uint32_t));
    if (e != hipSuccess) return hip_fail(e, "cx_qcsr_hybrid_prepare: hipMalloc");
    hipLaunchKernelGGL(zero_two_words, dim3(1), dim3(1), 0, s, words);
    const float qmax = static_cast<float>((1u << m->bits) - 1u);
    hipLaunchKernelGGL(head_range_kernel, dim3((head_cols + 255u) / 256u), dim3(256), 0, s, m->column_scales,
                       m->column_offsets, m->decode_policy, head_cols, qmax, words);
    if (m->decode_policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET && m->row_offsets != nullptr && m->rows != 0u)
        hipLaunchKernelGGL(abs_max_kernel, dim3(std::min<std::uint32_t>((m->rows + 255u) / 256u, 4096u)), dim3(256), 0,
                           s, m->row_offsets, m->rows, words + 1);
    std::uint32_t host[2] = {0u, 0u};
    e = hipMemcpyAsync(host, words, sizeof(host), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(words);
    if (e != hipSuccess) return hip_fail(e, "cx_qcsr_hybrid_prepare");
    float bound, roff;
    std::memcpy(&bound, &host[0], 4);
    std::memcpy(&roff, &host[1], 4);
    if (!(bound + roff < kHeadValueLimit))
        return fail(CX_STATUS_UNSUPPORTED,
                    "cx_qcsr_hybrid_prepare: head genes decode to |x| >= 2^15, outside the exact fp16 split");
    // the panel is a 16-bit word permutation ([head/32][out_cols][32]); the Blocked-ELL packer
    // moves fp16 words as well as bf16
    rc = cx_bell_pack_rhs(rhs_f16, rhs_ld, head_cols, out_cols, head_panel, stream);
    return rc;
}

extern "C" int cx_qcsr_hybrid_workspace(const cx_qcsr_matrix *m, uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (m == nullptr || bytes == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_hybrid_workspace: null argument");
    const std::uint64_t partial = (static_cast<std::uint64_t>(m->rows) * 64u * 4u + 255u) & ~std::uint64_t{255u};
    *bytes = partial + static_cast<std::uint64_t>(m->rows) * 4u;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_spmm_fwd_hybrid(const cx_qcsr_matrix *m, uint32_t head_cols, const uint16_t *head_panel,
                                       const void *rhs, int64_t rhs_ld, int64_t out_cols, float *out,
                                       int64_t out_ld, const cx_spmm_epilogue *epilogue, void *workspace,
                                       uint64_t workspace_bytes, void *stream) {
    using namespace cx;
    clear_error();
    int rc = validate_hybrid(m, head_cols, "cx_qcsr_spmm_fwd_hybrid: null matrix");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (rhs == nullptr || out == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_hybrid: null rhs or output");
    if (out_cols <= 0 || out_cols % 64 != 0 || out_cols > 256 || rhs_ld < out_cols || out_ld < out_cols)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_fwd_hybrid: out_cols must be 64, 128, 192 or 256");
    if ((m->flags & CX_QCSR_COLUMNS_SORTED) == 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_spmm_fwd_hybrid: rows must be sorted (CX_QCSR_COLUMNS_SORTED, e.g. from cx_qcsr_to_execution_order)");
    const bool aligned = (reinterpret_cast<std::uintptr_t>(rhs) & 15u) == 0u
        && (reinterpret_cast<std::uintptr_t>(out) & 15u) == 0u && (rhs_ld * 2) % 16 == 0 && (out_ld * 4) % 16 == 0;
    if (!aligned || m->cols > static_cast<std::uint32_t>(INT32_MAX) || rhs_ld > (INT32_MAX / 2) / 1024)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_hybrid: rhs and output must be 16-byte aligned");
    if (m->nnz > static_cast<std::uint64_t>(INT32_MAX))
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_fwd_hybrid: nnz exceeds int32 row offsets");
    if (static_cast<const void *>(out) == rhs)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_fwd_hybrid: output aliases the rhs");
    if (m->rows == 0u) return CX_STATUS_SUCCESS;
    Epilogue ep;
    rc = make_epilogue(epilogue, m->rows, out_cols, out, out_ld, &ep, "cx_qcsr_spmm_fwd_hybrid");
    if (rc != CX_STATUS_SUCCESS) return rc;
    std::uint64_t need = 0u;
    (void)cx_qcsr_hybrid_workspace(m, &need);
    if (head_cols != 0u && (workspace == nullptr || workspace_bytes < need || head_panel == nullptr
                            || (reinterpret_cast<std::uintptr_t>(workspace) & 255u) != 0u))
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_spmm_fwd_hybrid: needs the head panel and a 256-byte aligned workspace of cx_qcsr_hybrid_workspace bytes");
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
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (head_cols == 0u) return launch_qcsr_parts(a, m->bits, m->decode_policy, out_cols, s);
    auto *partial = static_cast<float *>(workspace);
    const std::uint64_t partial_bytes = (static_cast<std::uint64_t>(m->rows) * 64u * 4u + 255u) & ~std::uint64_t{255u};
    auto *head_end = reinterpret_cast<std::int32_t *>(static_cast<unsigned char *>(workspace) + partial_bytes);
    for (std::int64_t c0 = 0; c0 < out_cols; c0 += 64) {
        QcsrArgs b = a;
        rc = launch_qcsr_head(b, m->bits, m->decode_policy, head_cols, head_panel + c0 * 32,
                              static_cast<std::uint32_t>(out_cols), partial, head_end, s);
        if (rc != CX_STATUS_SUCCESS) return rc;
        b.rhs = static_cast<const std::uint16_t *>(rhs) + c0;
        b.out = out + c0;
        if (b.ep.bias != nullptr) b.ep.bias += c0;
        if (b.ep.initial != nullptr) b.ep.initial += c0;
        b.row_start = head_end;
        b.acc_init = partial;
        b.first_part = head_cols / 1024u;
        rc = launch_qcsr_parts(b, m->bits, m->decode_policy, 64, s);
        if (rc != CX_STATUS_SUCCESS) return rc;
    }
    return CX_STATUS_SUCCESS;
}
