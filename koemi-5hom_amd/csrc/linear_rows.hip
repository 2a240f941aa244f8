// Projections of a few rows (a decode step's 64 tokens) on bf16 MFMA.
//
// The HERM block's linear layers (nn.Linear in model/network.py and
// model/memory.py: the stacked working-state projections, the two gate
// projections, the fusion layer over [working ; memory ; local ; salient] of
// network.py:401-405 and the head) run on the libraries for a window of many
// rows. For a handful of rows a library GEMM is a long chain of dependent K
// steps over few workgroups, and each call needs the fp32 activations cast to
// bf16 (and the fusion input concatenated) by separate kernels first. Here one
// kernel streams the weights once: a workgroup owns 32 output features and up
// to 64 rows per pass (two 32-row MFMA blocks of v_mfma_f32_32x32x16_bf16).
// The input rows are staged in LDS as bf16, 1024 K values at a time, by
// coalesced 16-byte loads all issued at once (fp32 inputs rounded to nearest
// even on the way, as the cast they replace); each of the eight waves takes two
// 64-wide K steps of the chunk, its weight fragments loaded from global memory while the chunk is
// staged, and the waves add their partial sums through LDS at the end; the
// bias is added in the epilogue and the results are fp32. The input may be
// given as up to four row-major pieces of equal width that together form the
// K dimension (the concatenation is never built).
//
// Fragments use the MFMA register layout with a K permutation shared by both
// operands: lane l holds row l % 32 and, per step, the 32 contiguous values of
// half l / 32, of which MFMA j takes values 8j..8j+7, so every product pairs
// equal k.
#include "common.hpp"

#include <type_traits>

namespace koemi {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kCols = 32;
constexpr int kWaves = 8;
constexpr int kBlocks = 2;  // 32-row MFMA blocks per pass
constexpr int64_t kMaxRows = 64;

struct Pieces {
    const void* p[4];
};

// K values of the input staged in LDS at a time: sixteen 64-wide steps, two
// per wave, for bf16 inputs (all of K for the 1024-wide layers, so one memory
// round trip); eight for fp32 inputs, whose staging loads take twice the
// registers. Rows are padded by 16 bytes so that the 16-byte fragment reads of
// 16 consecutive rows fall in distinct banks. The cross-wave sums reuse the
// staging area once the last chunk is multiplied.
constexpr int kMaxChunk = 2 * kWaves * 64;
template <typename XT>
constexpr int chunk_of() { return sizeof(XT) == 2 ? kMaxChunk : kMaxChunk / 2; }
constexpr int kRowPitch = kMaxChunk + 8;  // bf16 elements
constexpr int kStageBytes = kBlocks * 32 * kRowPitch * 2;
constexpr int kRedBytes = kWaves * kBlocks * 16 * kWave * 4;
static_assert(kRedBytes <= kStageBytes, "the partial sums fit in the staging area");

// Independent projections of the same shape in one launch (a decode step's
// content heads of every layer): with a RowsBatch, blockIdx.y picks entry e,
// whose input (one piece), weight and bias replace the arguments and whose
// output is block e of y ([M, N] blocks one after another).
constexpr int kMaxBatch = 32;
struct RowsBatch {
    const void* x[kMaxBatch];
    const bf16* w[kMaxBatch];
    const float* bias[kMaxBatch];
};
struct NoBatch {};

// The gate projections of a decode step with the gates and the one-position
// scan in the epilogue (memory.py:14-30 with network.py:306-310): weight
// rows [0, F) are the retention projection, [F, 2F) the candidate one; a
// workgroup takes features [16 x, 16 x + 16) as its 32 MFMA columns (16
// retention rows, then the 16 matching candidate rows), and the thread of
// feature f finishes it: h = a h0 + b with (a, b) = gate_pair of the two
// sums (no GEMM bias; the gate biases and the validity inside gate_pair),
// as koemi_gated_scan does at one position.
struct NoGates {};
struct GatedStep {
    const float* retention_bias;  // [F] or null
    const float* candidate_bias;  // [F] or null
    const uint8_t* valid;         // [rows] or null
    const float* h0;              // [rows, F]
    float* h;                     // [rows, F]
    bf16* h16;                    // bf16 copy of h, rows h16_stride apart, or null
    int64_t h16_stride;
    int64_t F;
};

// Split K (k_len < K, no RowsBatch): blockIdx.y = split s takes K values
// [s k_len, (s + 1) k_len) and writes its partial sums to block s of y
// ([M, N] blocks one after another), the bias added by split 0 only; the
// consumer adds the blocks in split order.
template <typename XT, typename Batch = NoBatch, typename Gates = NoGates>
__global__ __launch_bounds__(kWaves * kWave) void linear_rows_kernel(Pieces in, int64_t piece_width,
                                                                     const bf16* __restrict__ w,
                                                                     const float* __restrict__ bias,
                                                                     float* __restrict__ y, int64_t M, int64_t N,
                                                                     int64_t K, Batch batch, int64_t k_len,
                                                                     Gates gates = Gates{}) {
    constexpr bool kGated = std::is_same<Gates, GatedStep>::value;
    int64_t k_begin = 0, k_end = K;
    if constexpr (std::is_same<Batch, RowsBatch>::value) {
        const int e = blockIdx.y;
        in = Pieces{{batch.x[e], batch.x[e], batch.x[e], batch.x[e]}};
        piece_width = K;
        w = batch.w[e];
        bias = batch.bias[e];
        y += static_cast<int64_t>(e) * M * N;
    } else {
        const int64_t split = blockIdx.y;
        k_begin = split * k_len;
        k_end = k_begin + k_len;
        y += split * M * N;
        if (split > 0) bias = nullptr;
    }
    __shared__ bf16x8 xs_raw[kStageBytes / 16];
    bf16* xs = reinterpret_cast<bf16*>(xs_raw);
    auto red = reinterpret_cast<float (*)[kBlocks][16][kWave]>(xs_raw);  // [kWaves][kBlocks][16][kWave]
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kCols;
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const int r = lane % 32, half = lane / 32;
    int64_t wn = n0 + r < N ? n0 + r : N - 1;  // rows past N are loaded from the last row, never stored
    if constexpr (kGated) {
        const int64_t f = static_cast<int64_t>(blockIdx.x) * 16 + r % 16;
        wn = (r < 16 ? 0 : gates.F) + (f < gates.F ? f : gates.F - 1);
    }
    const bf16* wr = w + wn * K + 32 * half;
    constexpr int kVec = 16 / sizeof(XT);  // input elements per 16-byte load
    constexpr int kChunk = chunk_of<XT>();
    // gated epilogue: this thread's carried states, validity and biases,
    // loaded before the partial sums go through LDS (their latency hides
    // under the exchange)
    constexpr int kEpi = kBlocks * 16 / kWaves;  // epilogue entries per thread
    float pre_h0[kEpi], pre_br = 0.0f, pre_bc = 0.0f;
    bool pre_keep[kEpi];
    auto preload = [&](int64_t pass) {
        if constexpr (kGated) {
            const int64_t f = static_cast<int64_t>(blockIdx.x) * 16 + lane % 32;
            const int64_t fc = f < gates.F ? f : gates.F - 1;
            pre_br = gates.retention_bias ? gates.retention_bias[fc] : 0.0f;
            pre_bc = gates.candidate_bias ? gates.candidate_bias[fc] : 0.0f;
#pragma unroll
            for (int q = 0; q < kEpi; ++q) {
                const int idx = q * kWaves + wave;
                const int64_t row = (idx / 16) * 32 + 8 * ((idx % 16) / 4) + 4 * (lane / 32) + (idx % 16) % 4;
                const int64_t br = pass + row < M ? pass + row : M - 1;
                pre_h0[q] = gates.h0[br * gates.F + fc];
                pre_keep[q] = gates.valid == nullptr || gates.valid[br] != 0;
            }
        }
    };
    for (int64_t pass = 0; pass < M; pass += kBlocks * 32) {
        const int64_t rows = M - pass < kBlocks * 32 ? M - pass : kBlocks * 32;
        const int blocks = rows > 32 ? 2 : 1;
        f32x16 acc[kBlocks];
#pragma unroll
        for (int rb = 0; rb < kBlocks; ++rb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rb][i] = 0.0f;
        for (int64_t c0 = k_begin; c0 < k_end; c0 += kChunk) {
            const int64_t ck = k_end - c0 < kChunk ? k_end - c0 : kChunk;  // a multiple of 64
            // This wave's weight fragments first (steps wave and wave + 8 of
            // the chunk), so that they load under the staging.
            bf16x8 wf[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int64_t kw = 64 * (wave + h * kWaves);
                if (kw < ck) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) wf[h][j] = *reinterpret_cast<const bf16x8*>(wr + c0 + kw + 8 * j);
                }
            }
            // Stage rows [pass, pass + rows) x k [c0, c0 + ck) as bf16: one
            // 16-byte input load per thread and iteration, consecutive threads
            // on consecutive addresses. A load never crosses a piece boundary
            // (piece_width is a multiple of 64), so its piece is looked up per load.
            // All of a thread's loads are issued before any is used (a fixed,
            // unrolled count), so the staging costs one memory round trip. A
            // chunk lies inside one piece (piece_width is a multiple of the
            // chunk, or there is one piece), so the piece is found once.
            constexpr int kPerRow = kChunk / kVec;  // 16-byte loads per staged row
            constexpr int kLoads = kBlocks * 32 * kPerRow / (kWaves * kWave);
            using Raw = typename std::conditional<sizeof(XT) == 2, bf16x8, float4>::type;
            Raw buf[kLoads];
            const int64_t piece = c0 / piece_width;
            const XT* base = static_cast<const XT*>(in.p[piece]) + pass * piece_width + (c0 - piece * piece_width);
            // Unconditional loads (positions past the rows or the chunk read a
            // valid element and land in staging slots nothing reads), so that
            // no branch separates them and they are all in flight together.
            const int last_row = static_cast<int>(rows) - 1, last_k = static_cast<int>(ck) - kVec;
#pragma unroll
            for (int u = 0; u < kLoads; ++u) {
                const int v = tid + u * kWaves * kWave;
                const int row = min(v / kPerRow, last_row), kk = min((v % kPerRow) * kVec, last_k);
                buf[u] = *reinterpret_cast<const Raw*>(base + row * piece_width + kk);
            }
#pragma unroll
            for (int u = 0; u < kLoads; ++u) {
                const int v = tid + u * kWaves * kWave;
                bf16* dst = xs + (v / kPerRow) * kRowPitch + (v % kPerRow) * kVec;
                if constexpr (sizeof(XT) == 2) {
                    *reinterpret_cast<bf16x8*>(dst) = buf[u];
                } else {
                    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
                    bf16x4 o;
                    o[0] = static_cast<__bf16>(buf[u].x);
                    o[1] = static_cast<__bf16>(buf[u].y);
                    o[2] = static_cast<__bf16>(buf[u].z);
                    o[3] = static_cast<__bf16>(buf[u].w);
                    *reinterpret_cast<bf16x4*>(dst) = o;
                }
            }
            __syncthreads();
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int kw = 64 * (wave + h * kWaves);
                if (kw >= ck) continue;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int rb = 0; rb < kBlocks; ++rb) {
                        if (rb >= blocks) continue;
                        const int row = rb * 32 + r;
                        bf16x8 xf = {};
                        if (row < rows) xf = *reinterpret_cast<const bf16x8*>(xs + row * kRowPitch + kw + 32 * half + 8 * j);
                        acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf, wf[h][j], acc[rb], 0, 0, 0);
                    }
            }
            __syncthreads();  // the staging area is rewritten by the next chunk (or holds the sums)
        }
        preload(pass);
#pragma unroll
        for (int rb = 0; rb < kBlocks; ++rb)
#pragma unroll
            for (int i = 0; i < 16; ++i) red[wave][rb][i][lane] = acc[rb][i];
        __syncthreads();
        // 2 blocks x 16 accumulator entries x 64 lanes, four per thread; entry i
        // of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4 of its block, column l % 32.
#pragma unroll
        for (int q = 0; q < kBlocks * 16 / kWaves; ++q) {
            const int idx = q * kWaves + wave;  // (block, entry), wave-uniform
            const int rb = idx / 16, i = idx % 16;
            const int64_t row = rb * 32 + 8 * (i / 4) + 4 * (lane / 32) + i % 4;
            if constexpr (kGated) {
                // lane c < 16 (of its half) holds retention feature 16 x + c, lane c + 16 its candidate
                const int64_t f = static_cast<int64_t>(blockIdx.x) * 16 + lane % 32;
                if (rb >= blocks || row >= rows || lane % 32 >= 16 || f >= gates.F) continue;
                float zr = 0.0f, zc = 0.0f;
#pragma unroll
                for (int w2 = 0; w2 < kWaves; ++w2) {
                    zr += red[w2][rb][i][lane];
                    zc += red[w2][rb][i][lane + 16];
                }
                const int64_t br = pass + row;
                float a, b;
                gate_pair(zr, zc, pre_br, pre_bc, pre_keep[q], a, b);
                const float hv = a * pre_h0[q] + b;
                gates.h[br * gates.F + f] = hv;
                if (gates.h16 != nullptr) gates.h16[br * gates.h16_stride + f] = static_cast<__bf16>(hv);
                continue;
            }
            const int64_t col = n0 + lane % 32;
            if (rb >= blocks || row >= rows || col >= N) continue;
            float v = bias != nullptr ? bias[col] : 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < kWaves; ++w2) v += red[w2][rb][i][lane];
            y[(pass + row) * N + col] = v;
        }
        __syncthreads();  // red is rewritten by the next pass
    }
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" int koemi_linear_rows(const void* input0, const void* input1, const void* input2, const void* input3,
                                 int pieces, int64_t piece_width, int input_dtype, const void* weight,
                                 const float* bias, float* output, int64_t rows, int64_t out_features,
                                 koemi_stream_t stream) {
    if (rows < 0 || out_features < 1 || piece_width < 1 || pieces < 1 || pieces > 4)
        return fail(KOEMI_ERR_INVALID, "linear rows needs rows >= 0, 1 to 4 input pieces and positive widths");
    if (input_dtype != KOEMI_F32 && input_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows takes float32 or bfloat16 inputs, not %s",
                    dtype_name(input_dtype));
    if (piece_width % 64 != 0 || (pieces > 1 && piece_width % kMaxChunk != 0))
        return fail(KOEMI_ERR_UNSUPPORTED,
                    "linear rows needs an input width that is a multiple of 64 (of 1024 for several pieces)");
    if (rows > kMaxRows * 1024 || out_features > 0x7fffffffLL / 2)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows is for a few rows (at most %lld)",
                    static_cast<long long>(kMaxRows * 1024));
    if (rows == 0) return KOEMI_OK;
    const void* in[4] = {input0, input1, input2, input3};
    const size_t elem = input_dtype == KOEMI_F32 ? 4 : 2;
    for (int i = 0; i < pieces; ++i)
        if (!in[i] || reinterpret_cast<uintptr_t>(in[i]) % (8 * elem) != 0)
            return fail(KOEMI_ERR_INVALID, "linear rows input %d is null or not %zu-byte aligned", i, 8 * elem);
    if (!weight || reinterpret_cast<uintptr_t>(weight) % 16 != 0 || !output)
        return fail(KOEMI_ERR_INVALID, "linear rows needs a 16-byte aligned weight and an output");
    const Pieces p{{in[0], pieces > 1 ? in[1] : in[0], pieces > 2 ? in[2] : in[0], pieces > 3 ? in[3] : in[0]}};
    const int64_t K = piece_width * pieces;
    const dim3 grid(static_cast<unsigned>((out_features + kCols - 1) / kCols)), block(kWaves * kWave);
    const hipStream_t s = as_stream(stream);
    if (input_dtype == KOEMI_F32)
        hipLaunchKernelGGL(linear_rows_kernel<float>, grid, block, 0, s, p, piece_width,
                           static_cast<const bf16*>(weight), bias, output, rows, out_features, K, NoBatch{}, K, NoGates{});
    else
        hipLaunchKernelGGL(linear_rows_kernel<bf16>, grid, block, 0, s, p, piece_width,
                           static_cast<const bf16*>(weight), bias, output, rows, out_features, K, NoBatch{}, K, NoGates{});
    return check_launch("koemi_linear_rows");
}

extern "C" int koemi_linear_rows_gated(const void* input, int input_dtype, const void* weight,
                                       const float* retention_bias, const float* candidate_bias,
                                       const uint8_t* valid, const float* initial, float* states, void* states_bf16,
                                       int64_t bf16_row_stride, int64_t rows, int64_t width, int64_t in_features,
                                       koemi_stream_t stream) {
    if (rows < 0 || width < 1 || in_features < 1)
        return fail(KOEMI_ERR_INVALID, "gated linear rows needs rows >= 0 and positive widths");
    if (input_dtype != KOEMI_F32 && input_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows takes float32 or bfloat16 inputs, not %s",
                    dtype_name(input_dtype));
    if (in_features % 64 != 0)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows needs an input width that is a multiple of 64");
    if (rows > kMaxRows * 1024 || width > 0x7fffffffLL / 32)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows is for a few rows (at most %lld)",
                    static_cast<long long>(kMaxRows * 1024));
    if (states_bf16 != nullptr && bf16_row_stride < width)
        return fail(KOEMI_ERR_INVALID, "gated linear rows: the bf16 row stride is below the width");
    if (rows == 0) return KOEMI_OK;
    const size_t elem = input_dtype == KOEMI_F32 ? 4 : 2;
    if (!input || reinterpret_cast<uintptr_t>(input) % (8 * elem) != 0 || !weight ||
        reinterpret_cast<uintptr_t>(weight) % 16 != 0 || !initial || !states)
        return fail(KOEMI_ERR_INVALID, "gated linear rows received a null or unaligned pointer");
    const Pieces p{{input, input, input, input}};
    const GatedStep g{retention_bias, candidate_bias, valid, initial, states, static_cast<bf16*>(states_bf16),
                      bf16_row_stride, width};
    const dim3 grid(static_cast<unsigned>((width + 15) / 16));
    const hipStream_t s = as_stream(stream);
    const float* none = nullptr;
    if (input_dtype == KOEMI_F32)
        hipLaunchKernelGGL((linear_rows_kernel<float, NoBatch, GatedStep>), grid, dim3(kWaves * kWave), 0, s, p,
                           in_features, static_cast<const bf16*>(weight), none, states, rows, 2 * width,
                           in_features, NoBatch{}, in_features, g);
    else
        hipLaunchKernelGGL((linear_rows_kernel<bf16, NoBatch, GatedStep>), grid, dim3(kWaves * kWave), 0, s, p,
                           in_features, static_cast<const bf16*>(weight), none, states, rows, 2 * width,
                           in_features, NoBatch{}, in_features, g);
    return check_launch("koemi_linear_rows_gated");
}

extern "C" int koemi_linear_rows_split(const void* input0, const void* input1, const void* input2,
                                       const void* input3, int pieces, int64_t piece_width, int input_dtype,
                                       const void* weight, const float* bias, float* partials, int64_t rows,
                                       int64_t out_features, int splits, koemi_stream_t stream) {
    if (rows < 0 || out_features < 1 || piece_width < 1 || pieces < 1 || pieces > 4 || splits < 1)
        return fail(KOEMI_ERR_INVALID, "split linear rows needs rows >= 0, 1 to 4 pieces, positive widths and splits");
    if (input_dtype != KOEMI_F32 && input_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows takes float32 or bfloat16 inputs, not %s",
                    dtype_name(input_dtype));
    const int64_t K = piece_width * pieces;
    const int64_t chunk = input_dtype == KOEMI_F32 ? chunk_of<float>() : chunk_of<bf16>();
    if (piece_width % kMaxChunk != 0 || K % splits != 0 || (K / splits) % chunk != 0 || splits > 65535)
        return fail(KOEMI_ERR_UNSUPPORTED,
                    "split linear rows needs pieces of a multiple of 1024 and K / splits a multiple of %lld",
                    static_cast<long long>(chunk));
    if (rows > kMaxRows * 1024 || out_features > 0x7fffffffLL / 2)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows is for a few rows (at most %lld)",
                    static_cast<long long>(kMaxRows * 1024));
    if (rows == 0) return KOEMI_OK;
    const void* in[4] = {input0, input1, input2, input3};
    const size_t elem = input_dtype == KOEMI_F32 ? 4 : 2;
    for (int i = 0; i < pieces; ++i)
        if (!in[i] || reinterpret_cast<uintptr_t>(in[i]) % (8 * elem) != 0)
            return fail(KOEMI_ERR_INVALID, "linear rows input %d is null or not %zu-byte aligned", i, 8 * elem);
    if (!weight || reinterpret_cast<uintptr_t>(weight) % 16 != 0 || !partials)
        return fail(KOEMI_ERR_INVALID, "linear rows needs a 16-byte aligned weight and an output");
    const Pieces p{{in[0], pieces > 1 ? in[1] : in[0], pieces > 2 ? in[2] : in[0], pieces > 3 ? in[3] : in[0]}};
    const dim3 grid(static_cast<unsigned>((out_features + kCols - 1) / kCols), static_cast<unsigned>(splits));
    const hipStream_t s = as_stream(stream);
    if (input_dtype == KOEMI_F32)
        hipLaunchKernelGGL(linear_rows_kernel<float>, grid, dim3(kWaves * kWave), 0, s, p, piece_width,
                           static_cast<const bf16*>(weight), bias, partials, rows, out_features, K, NoBatch{},
                           K / splits, NoGates{});
    else
        hipLaunchKernelGGL(linear_rows_kernel<bf16>, grid, dim3(kWaves * kWave), 0, s, p, piece_width,
                           static_cast<const bf16*>(weight), bias, partials, rows, out_features, K, NoBatch{},
                           K / splits, NoGates{});
    return check_launch("koemi_linear_rows_split");
}

extern "C" int koemi_linear_rows_batched(const void* const* inputs, int input_dtype, const void* const* weights,
                                         const float* const* biases, float* output, int count, int64_t rows,
                                         int64_t in_features, int64_t out_features, koemi_stream_t stream) {
    if (count < 1 || rows < 0 || out_features < 1 || in_features < 1)
        return fail(KOEMI_ERR_INVALID, "batched linear rows needs count >= 1, rows >= 0 and positive widths");
    if (count > kMaxBatch)
        return fail(KOEMI_ERR_UNSUPPORTED, "batched linear rows takes at most %d projections", kMaxBatch);
    if (input_dtype != KOEMI_F32 && input_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows takes float32 or bfloat16 inputs, not %s",
                    dtype_name(input_dtype));
    if (in_features % 64 != 0)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows needs an input width that is a multiple of 64");
    if (rows > kMaxRows * 1024 || out_features > 0x7fffffffLL / 2)
        return fail(KOEMI_ERR_UNSUPPORTED, "linear rows is for a few rows (at most %lld)",
                    static_cast<long long>(kMaxRows * 1024));
    if (rows == 0) return KOEMI_OK;
    if (!inputs || !weights || !output) return fail(KOEMI_ERR_INVALID, "batched linear rows received a null pointer");
    const size_t elem = input_dtype == KOEMI_F32 ? 4 : 2;
    RowsBatch b{};
    for (int e = 0; e < count; ++e) {
        if (!inputs[e] || reinterpret_cast<uintptr_t>(inputs[e]) % (8 * elem) != 0 || !weights[e] ||
            reinterpret_cast<uintptr_t>(weights[e]) % 16 != 0)
            return fail(KOEMI_ERR_INVALID, "batched linear rows: projection %d has a null or unaligned operand", e);
        b.x[e] = inputs[e];
        b.w[e] = static_cast<const bf16*>(weights[e]);
        b.bias[e] = biases != nullptr ? biases[e] : nullptr;
    }
    const Pieces none{{nullptr, nullptr, nullptr, nullptr}};
    const dim3 grid(static_cast<unsigned>((out_features + kCols - 1) / kCols), static_cast<unsigned>(count));
    const hipStream_t s = as_stream(stream);
    if (input_dtype == KOEMI_F32)
        hipLaunchKernelGGL((linear_rows_kernel<float, RowsBatch>), grid, dim3(kWaves * kWave), 0, s, none,
                           in_features, static_cast<const bf16*>(nullptr), static_cast<const float*>(nullptr), output,
                           rows, out_features, in_features, b, in_features, NoGates{});
    else
        hipLaunchKernelGGL((linear_rows_kernel<bf16, RowsBatch>), grid, dim3(kWaves * kWave), 0, s, none,
                           in_features, static_cast<const bf16*>(nullptr), static_cast<const float*>(nullptr), output,
                           rows, out_features, in_features, b, in_features, NoGates{});
    return check_launch("koemi_linear_rows_batched");
}
