// Small per-window steps of the HERM block for gfx950 (torch composites in
// the reference), each one kernel:
//
//   koemi_herm_rmsnorm: RootMeanSquareNorm (layers.py:14-16) of x (+ an
//     optional residual), kept only on rows whose mask byte is set (others
//     copy x): the input normalizer (network.py:703-707), the fusion normalizer
//     (network.py:723-732) and the expert mixture's output normalizer with its
//     valid-row select (experts.py:134-136). One wave per row, the row in
//     registers, fp32 sum of squares, 16-byte loads.
//   koemi_herm_token_context: the previous valid token of each position and
//     the last valid token of each row (network.py:742-761). One workgroup per
//     row, a max-scan of the valid positions.
//   koemi_herm_concat_bf16: the fusion layer's input [working ; memory ;
//     local ; salient] (network.py:401-405) as one bf16 matrix for its GEMM,
//     the concatenation and the cast in one pass.
#include "common.hpp"

namespace koemi {
namespace {

template <typename X, typename R, int NV>
__global__ __launch_bounds__(256) void herm_rmsnorm_kernel(const X* __restrict__ x, const R* __restrict__ residual,
                                                           const float* __restrict__ w,
                                                           const uint8_t* __restrict__ mask, float* __restrict__ y,
                                                           bf16* __restrict__ y16, int64_t rows, int H, float eps) {
    const int lane = lane_id();
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (row >= rows) return;
    const X* xr = x + row * H;
    float v[NV][4];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * kWave + lane) * 4;
        if (c < H) {
            const float4 q = load4(xr + c);
            v[j][0] = q.x; v[j][1] = q.y; v[j][2] = q.z; v[j][3] = q.w;
            if (residual != nullptr) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[j][i] += to_f32(residual[row * H + c + i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[j][i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) ss = fmaf(v[j][i], v[j][i], ss);
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, kWave);
    const bool keep = mask == nullptr || mask[row] != 0;
    const float inv = rsqrtf(ss / static_cast<float>(H) + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * kWave + lane) * 4;
        if (c >= H) continue;
        float4 o;
        if (keep) {
            const float4 wq = *reinterpret_cast<const float4*>(w + c);
            o = make_float4(v[j][0] * inv * wq.x, v[j][1] * inv * wq.y, v[j][2] * inv * wq.z, v[j][3] * inv * wq.w);
        } else {
            o = load4(xr + c);
        }
        if (y != nullptr) *reinterpret_cast<float4*>(y + row * H + c) = o;
        if (y16 != nullptr) {
            typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
            bf16x4 q;
            q[0] = static_cast<__bf16>(o.x); q[1] = static_cast<__bf16>(o.y);
            q[2] = static_cast<__bf16>(o.z); q[3] = static_cast<__bf16>(o.w);
            *reinterpret_cast<bf16x4*>(y16 + row * H + c) = q;
        }
    }
}

// koemi_herm_rmsnorm_parts: one workgroup per row, thread t on columns
// 4 t + 1024 i. The input is the sum of `parts` fp32 blocks part_stride
// elements apart, added in block order (a split projection's partial sums;
// every block's load issued before the sums), plus add_bias, optionally
// rounded to bf16; the row's sum of squares is reduced over the wave, then
// over the four waves in order.
constexpr int kMaxParts = 8;

template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_parts_kernel(const float* __restrict__ x, int parts,
                                                            int64_t part_stride, const float* __restrict__ add_bias,
                                                            int round16, const float* __restrict__ w,
                                                            float* __restrict__ y, bf16* __restrict__ y16, int H,
                                                            float eps) {
    __shared__ float wave_ss[4];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const float* xr = x + row * H;
    float v[NV][4];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * 256 + tid) * 4;
        if (c < H) {
            float4 r4[kMaxParts];
#pragma unroll
            for (int pt = 0; pt < kMaxParts; ++pt) r4[pt] = load4(xr + min(pt, parts - 1) * part_stride + c);
            v[j][0] = r4[0].x; v[j][1] = r4[0].y; v[j][2] = r4[0].z; v[j][3] = r4[0].w;
#pragma unroll
            for (int pt = 1; pt < kMaxParts; ++pt) {
                const bool on = pt < parts;
                v[j][0] += on ? r4[pt].x : 0.0f; v[j][1] += on ? r4[pt].y : 0.0f;
                v[j][2] += on ? r4[pt].z : 0.0f; v[j][3] += on ? r4[pt].w : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (add_bias != nullptr) v[j][i] += add_bias[c + i];
                if (round16) v[j][i] = static_cast<float>(static_cast<__bf16>(v[j][i]));
                ss = fmaf(v[j][i], v[j][i], ss);
            }
        }
    }
    ss = wave_sum_xor(ss);
    if (lane == 0) wave_ss[wave] = ss;
    __syncthreads();
    const float total = ((wave_ss[0] + wave_ss[1]) + wave_ss[2]) + wave_ss[3];
    const float inv = rsqrtf(total / static_cast<float>(H) + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * 256 + tid) * 4;
        if (c >= H) continue;
        const float4 wq = *reinterpret_cast<const float4*>(w + c);
        const float4 o = make_float4(v[j][0] * inv * wq.x, v[j][1] * inv * wq.y, v[j][2] * inv * wq.z,
                                     v[j][3] * inv * wq.w);
        if (y != nullptr) *reinterpret_cast<float4*>(y + row * H + c) = o;
        if (y16 != nullptr) {
            typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
            bf16x4 q;
            q[0] = static_cast<__bf16>(o.x); q[1] = static_cast<__bf16>(o.y);
            q[2] = static_cast<__bf16>(o.z); q[3] = static_cast<__bf16>(o.w);
            *reinterpret_cast<bf16x4*>(y16 + row * H + c) = q;
        }
    }
}

// Greedy next tokens: one wave per row, the first maximum of the row with
// `exclude` scored -inf (a NaN counts as the maximum, as torch.argmax treats
// it); each lane scans columns lane, lane + 64, ..., then a shuffle
// reduction keeps the better (value, index) pair, ties to the lower index.
__device__ __forceinline__ bool greedy_better(float av, int64_t ai, float bv, int64_t bi) {
    const bool an = av != av, bn = bv != bv;
    if (an != bn) return an;
    if (!an && av != bv) return av > bv;
    return ai < bi;
}

__global__ __launch_bounds__(256) void greedy_tokens_kernel(const float* __restrict__ logits, int64_t row_stride,
                                                            int64_t rows, int64_t V, int64_t exclude,
                                                            int64_t* __restrict__ ids) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (row >= rows) return;
    const int lane = lane_id();
    const float* z = logits + row * row_stride;
    float bv = -INFINITY;
    int64_t bi = V;  // past every column: loses every comparison
    for (int64_t j = lane; j < V; j += kWave) {
        const float v = j == exclude ? -INFINITY : z[j];
        if (greedy_better(v, j, bv, bi)) {
            bv = v;
            bi = j;
        }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, kWave);
        const int64_t oi = __shfl_xor(bi, off, kWave);
        if (greedy_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) ids[row] = bi < V ? bi : 0;
}

// TokenSampler's non-greedy draw (runtime/fast_decode.py:57-95): one
// workgroup per row of fp32 scores (column `exclude`, the PAD id, at -inf),
// kept = min(top_k, V) and, when kept < V, every score below the kept-th
// largest (duplicates counted, ties kept) set to -inf; y = score /
// temperature; p = softmax(y) (max, exp, sum in a fixed order); the draw is
// the first column whose cumulative probability (in column order) exceeds the
// row's uniform u in [0, 1), or, when rounding leaves u at or above the last
// cumulative value, the last column with p > 0. `probs` (null: none) receives
// p. The caller supplies the uniforms, so a captured graph draws
// reproducibly from whatever random numbers it is given.
constexpr int kSampleThreads = 256;
constexpr int kSampleMaxV = 4096;

__device__ __forceinline__ float block_reduce(float v, float* sh, bool is_max) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float o = __shfl_xor(v, off, kWave);
        v = is_max ? fmaxf(v, o) : v + o;
    }
    __syncthreads();  // sh may still be read from an earlier reduction
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float r = sh[0];
    for (int w = 1; w < kSampleThreads / kWave; ++w) r = is_max ? fmaxf(r, sh[w]) : r + sh[w];
    return r;
}

__global__ __launch_bounds__(kSampleThreads) void sample_tokens_kernel(
    const float* __restrict__ logits, int64_t row_stride, int64_t V, int64_t exclude, float temperature,
    int64_t top_k, const float* __restrict__ uniforms, int64_t* __restrict__ ids, float* __restrict__ probs) {
    __shared__ float sc[kSampleMaxV];
    __shared__ float red[kSampleThreads / kWave];
    __shared__ float thr_sh;
    __shared__ float scan_sh[kSampleThreads];
    __shared__ int first_sh, last_sh;
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* z = logits + row * row_stride;
    for (int64_t j = tid; j < V; j += kSampleThreads) sc[j] = j == exclude ? -INFINITY : z[j];
    if (tid == 0) {
        thr_sh = -INFINITY;
        first_sh = static_cast<int>(V);
        last_sh = -1;
    }
    __syncthreads();
    const int64_t kept = top_k > 0 ? (top_k < V ? top_k : V) : V;
    if (kept < V) {
        for (int64_t j = tid; j < V; j += kSampleThreads) {
            const float x = sc[j];
            int64_t gt = 0, ge = 0;
            for (int64_t i = 0; i < V; ++i) {
                gt += sc[i] > x;
                ge += sc[i] >= x;
            }
            if (gt < kept && ge >= kept) thr_sh = x;  // every such column holds the same value
        }
    }
    __syncthreads();
    const float thr = thr_sh;
    float mx = -INFINITY;
    for (int64_t j = tid; j < V; j += kSampleThreads) {
        const float y = (sc[j] < thr ? -INFINITY : sc[j]) / temperature;
        sc[j] = y;
        mx = fmaxf(mx, y);
    }
    mx = block_reduce(mx, red, true);
    float sum = 0.0f;
    for (int64_t j = tid; j < V; j += kSampleThreads) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    sum = block_reduce(sum, red, false);
    // probabilities, then the inverse CDF: thread t owns columns [t c, t c + c)
    const int64_t c = (V + kSampleThreads - 1) / kSampleThreads;
    const int64_t j0 = tid * c, j1 = j0 + c < V ? j0 + c : V;
    float local = 0.0f;
    for (int64_t j = j0; j < j1; ++j) {
        const float pj = sc[j] / sum;
        sc[j] = pj;
        local += pj;
        if (probs) probs[row * V + j] = pj;
    }
    scan_sh[tid] = local;
    __syncthreads();
    if (tid == 0) {  // exclusive prefix of the threads' sums, in column order
        float run = 0.0f;
        for (int t = 0; t < kSampleThreads; ++t) {
            const float v = scan_sh[t];
            scan_sh[t] = run;
            run += v;
        }
    }
    __syncthreads();
    const float u = uniforms[row];
    float cum = scan_sh[tid];
    for (int64_t j = j0; j < j1; ++j) {
        cum += sc[j];
        if (cum > u) {
            atomicMin(&first_sh, static_cast<int>(j));
            break;
        }
    }
    for (int64_t j = j1 - 1; j >= j0; --j)
        if (sc[j] > 0.0f) {
            atomicMax(&last_sh, static_cast<int>(j));
            break;
        }
    __syncthreads();
    if (tid == 0) ids[row] = first_sh < V ? first_sh : (last_sh >= 0 ? last_sh : 0);
}

// One workgroup per row: position t takes the latest valid index before it,
// an exclusive max-scan of (valid ? t : -1) over 256-position chunks (a wave
// scan, the wave maxima through LDS, the chunk's carry in a register).
// With `valid` null the validity is ids != pad_id, written to valid_out, and
// targets_out (if given) gets ids where valid, 0 elsewhere (network.py:335,
// the surprise targets).
__global__ __launch_bounds__(256) void herm_token_context_kernel(const int64_t* __restrict__ ids,
                                                                 const uint8_t* __restrict__ valid,
                                                                 const int64_t* __restrict__ carried,
                                                                 int64_t* __restrict__ previous,
                                                                 int64_t* __restrict__ last,
                                                                 uint8_t* __restrict__ valid_out,
                                                                 int64_t* __restrict__ targets_out, int64_t pad_id,
                                                                 int64_t L) {
    __shared__ int wave_max[4];
    const int64_t b = blockIdx.x;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    int carry = -1;  // latest valid index before the chunk
    for (int64_t c0 = 0; c0 < L; c0 += 256) {
        const int64_t t = c0 + tid;
        bool ok = false;
        if (t < L) {
            const int64_t id = ids[b * L + t];
            ok = valid != nullptr ? valid[b * L + t] != 0 : id != pad_id;
            if (valid_out != nullptr) valid_out[b * L + t] = ok ? 1 : 0;
            if (targets_out != nullptr) targets_out[b * L + t] = ok ? id : 0;
        }
        const int mine = ok ? static_cast<int>(t) : -1;
        int incl = mine;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int up = __shfl_up(incl, off, kWave);
            if (lane >= off) incl = max(incl, up);
        }
        if (lane == kWave - 1) wave_max[wave] = incl;
        __syncthreads();
        int before = carry;
        for (int w = 0; w < wave; ++w) before = max(before, wave_max[w]);
        const int left = __shfl_up(incl, 1, kWave);  // every lane takes part
        const int prev_index = lane > 0 ? max(before, left) : before;
        if (t < L) previous[b * L + t] = prev_index >= 0 ? ids[b * L + prev_index] : carried[b];
        int chunk_max = carry;
        for (int w = 0; w < 4; ++w) chunk_max = max(chunk_max, wave_max[w]);
        __syncthreads();
        carry = chunk_max;
    }
    if (tid == 0) last[b] = carry >= 0 ? ids[b * L + carry] : carried[b];
}

// [rows, pieces * width] bf16 from `pieces` fp32 [rows, width] blocks; a thread
// converts four consecutive values (16-byte load, 8-byte store).
struct ConcatPieces {
    const float* p[4];
};
__global__ __launch_bounds__(256) void herm_concat_bf16_kernel(ConcatPieces in, int pieces, int64_t rows,
                                                               int64_t width, bf16* __restrict__ out) {
    const int64_t quads = width / 4;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows * pieces * quads) return;
    const int64_t row = i / (pieces * quads);
    const int64_t rest = i - row * pieces * quads;
    const int piece = static_cast<int>(rest / quads);
    const int64_t c = (rest - piece * quads) * 4;
    const float4 v = *reinterpret_cast<const float4*>(in.p[piece] + row * width + c);
    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
    bf16x4 q;
    q[0] = static_cast<__bf16>(v.x); q[1] = static_cast<__bf16>(v.y);
    q[2] = static_cast<__bf16>(v.z); q[3] = static_cast<__bf16>(v.w);
    *reinterpret_cast<bf16x4*>(out + row * pieces * width + piece * width + c) = q;
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" int koemi_herm_rmsnorm(const void* input, int input_dtype, const void* residual, int residual_dtype,
                                  const float* weight, const uint8_t* mask, float* output, void* output_bf16,
                                  int64_t rows, int64_t width, float eps, koemi_stream_t stream) {
    if (rows < 0 || width < 1) return fail(KOEMI_ERR_INVALID, "herm rmsnorm needs rows >= 0 and a positive width");
    if (input_dtype != KOEMI_F32 && input_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "herm rmsnorm input dtype %s", dtype_name(input_dtype));
    if (width % 4 != 0 || width > 4 * kWave * 8)
        return fail(KOEMI_ERR_UNSUPPORTED, "herm rmsnorm needs a width that is a multiple of 4 and at most 2048");
    if (residual != nullptr && residual_dtype != KOEMI_F32 && residual_dtype != KOEMI_BF16 && residual_dtype != KOEMI_F16)
        return fail(KOEMI_ERR_UNSUPPORTED, "herm rmsnorm residual dtype %s", dtype_name(residual_dtype));
    if (rows == 0) return KOEMI_OK;
    if (!input || !weight || (!output && !output_bf16))
        return fail(KOEMI_ERR_INVALID, "herm rmsnorm received a null pointer");
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
    const hipStream_t s = as_stream(stream);
    const int H = static_cast<int>(width);
    auto launch = [&](auto xtag, auto tag) {
        using X = decltype(xtag);
        using R = decltype(tag);
        const X* x = static_cast<const X*>(input);
        const R* r = static_cast<const R*>(residual);
        bf16* o16 = static_cast<bf16*>(output_bf16);
        if (width <= 4 * kWave * 4)
            hipLaunchKernelGGL((herm_rmsnorm_kernel<X, R, 4>), grid, dim3(256), 0, s, x, r, weight, mask, output, o16,
                               rows, H, eps);
        else
            hipLaunchKernelGGL((herm_rmsnorm_kernel<X, R, 8>), grid, dim3(256), 0, s, x, r, weight, mask, output, o16,
                               rows, H, eps);
    };
    auto with_input = [&](auto tag) {
        if (input_dtype == KOEMI_BF16) launch(bf16{}, tag);
        else launch(float{}, tag);
    };
    if (residual == nullptr || residual_dtype == KOEMI_F32) with_input(float{});
    else if (residual_dtype == KOEMI_BF16) with_input(bf16{});
    else with_input(f16{});
    return check_launch("koemi_herm_rmsnorm");
}

extern "C" int koemi_herm_rmsnorm_parts(const float* parts_input, int parts, const float* add_bias, int round_bf16,
                                        const float* weight, float* output, void* output_bf16, int64_t rows,
                                        int64_t width, float eps, koemi_stream_t stream) {
    if (rows < 0 || width < 1 || parts < 1)
        return fail(KOEMI_ERR_INVALID, "herm rmsnorm parts needs rows >= 0, a positive width and parts >= 1");
    if (parts > kMaxParts) return fail(KOEMI_ERR_UNSUPPORTED, "herm rmsnorm parts adds at most %d blocks", kMaxParts);
    if (width % 4 != 0 || width > 2048)
        return fail(KOEMI_ERR_UNSUPPORTED, "herm rmsnorm needs a width that is a multiple of 4 and at most 2048");
    if (rows == 0) return KOEMI_OK;
    if (rows > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "herm rmsnorm parts: too many rows");
    if (!parts_input || !weight || (!output && !output_bf16) || reinterpret_cast<uintptr_t>(parts_input) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(weight) % 16 != 0)
        return fail(KOEMI_ERR_INVALID, "herm rmsnorm parts received a null or unaligned pointer");
    const int H = static_cast<int>(width);
    bf16* o16 = static_cast<bf16*>(output_bf16);
    const dim3 grid(static_cast<unsigned>(rows));
    if (width <= 1024)
        hipLaunchKernelGGL(rmsnorm_parts_kernel<1>, grid, dim3(256), 0, as_stream(stream), parts_input, parts,
                           rows * width, add_bias, round_bf16, weight, output, o16, H, eps);
    else
        hipLaunchKernelGGL(rmsnorm_parts_kernel<2>, grid, dim3(256), 0, as_stream(stream), parts_input, parts,
                           rows * width, add_bias, round_bf16, weight, output, o16, H, eps);
    return check_launch("koemi_herm_rmsnorm_parts");
}

extern "C" int koemi_herm_greedy_tokens(const float* logits, int64_t row_stride, int64_t rows, int64_t vocab,
                                        int64_t exclude_id, int64_t* ids, koemi_stream_t stream) {
    if (rows < 0 || vocab < 1 || row_stride < vocab)
        return fail(KOEMI_ERR_INVALID, "greedy tokens need rows >= 0, vocab >= 1 and row_stride >= vocab");
    if (rows == 0) return KOEMI_OK;
    if (!logits || !ids) return fail(KOEMI_ERR_INVALID, "greedy tokens received a null pointer");
    if ((rows + 3) / 4 > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "greedy tokens: too many rows");
    hipLaunchKernelGGL(greedy_tokens_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0,
                       as_stream(stream), logits, row_stride, rows, vocab, exclude_id, ids);
    return check_launch("koemi_herm_greedy_tokens");
}

extern "C" int koemi_herm_sample_tokens(const float* logits, int64_t row_stride, int64_t rows, int64_t vocab,
                                        int64_t exclude_id, float temperature, int64_t top_k, const float* uniforms,
                                        int64_t* ids, float* probabilities, koemi_stream_t stream) {
    if (rows < 0 || vocab < 1) return fail(KOEMI_ERR_INVALID, "token sampling needs rows >= 0 and a positive vocabulary");
    if (!(temperature > 0.0f)) return fail(KOEMI_ERR_INVALID, "temperature must be positive");
    if (top_k < 0) return fail(KOEMI_ERR_INVALID, "top_k must be a positive integer (0: none)");
    if (vocab > kSampleMaxV) return fail(KOEMI_ERR_UNSUPPORTED, "token sampling supports at most %d columns", kSampleMaxV);
    if (row_stride == 0) row_stride = vocab;
    if (row_stride < vocab) return fail(KOEMI_ERR_INVALID, "token sampling row stride below the vocabulary");
    if (rows == 0) return KOEMI_OK;
    if (!logits || !uniforms || !ids) return fail(KOEMI_ERR_INVALID, "token sampling received a null pointer");
    if (rows > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "token sampling: too many rows");
    hipLaunchKernelGGL(sample_tokens_kernel, dim3(static_cast<unsigned>(rows)), dim3(kSampleThreads), 0,
                       as_stream(stream), logits, row_stride, vocab, exclude_id, temperature, top_k, uniforms, ids,
                       probabilities);
    return check_launch("koemi_herm_sample_tokens");
}

extern "C" int koemi_herm_token_context(const int64_t* token_ids, const uint8_t* valid, const int64_t* carried_last,
                                        int64_t* previous, int64_t* last, uint8_t* valid_out, int64_t* targets_out,
                                        int64_t pad_id, int64_t batch, int64_t length, koemi_stream_t stream) {
    if (batch < 0 || length < 0) return fail(KOEMI_ERR_INVALID, "token context needs non-negative sizes");
    if (batch == 0) return KOEMI_OK;
    if (!token_ids || !carried_last || !previous || !last || (!valid && !valid_out))
        return fail(KOEMI_ERR_INVALID, "token context received a null pointer");
    if (batch > 0x7fffffffLL || length > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "token context sizes too large");
    hipLaunchKernelGGL(herm_token_context_kernel, dim3(static_cast<unsigned>(batch)), dim3(256), 0, as_stream(stream),
                       token_ids, valid, carried_last, previous, last, valid_out, targets_out, pad_id, length);
    return check_launch("koemi_herm_token_context");
}

extern "C" int koemi_herm_concat_bf16(const float* input0, const float* input1, const float* input2,
                                      const float* input3, int pieces, int64_t rows, int64_t width, void* output,
                                      koemi_stream_t stream) {
    if (pieces < 1 || pieces > 4 || rows < 0 || width < 1)
        return fail(KOEMI_ERR_INVALID, "concat needs 1 to 4 pieces, rows >= 0 and a positive width");
    if (width % 4 != 0) return fail(KOEMI_ERR_UNSUPPORTED, "concat needs a width that is a multiple of 4");
    if (rows == 0) return KOEMI_OK;
    const float* in[4] = {input0, input1, input2, input3};
    for (int i = 0; i < pieces; ++i)
        if (!in[i] || reinterpret_cast<uintptr_t>(in[i]) % 16 != 0)
            return fail(KOEMI_ERR_INVALID, "concat input %d is null or not 16-byte aligned", i);
    if (!output || reinterpret_cast<uintptr_t>(output) % 8 != 0)
        return fail(KOEMI_ERR_INVALID, "concat output is null or not 8-byte aligned");
    const int64_t threads = rows * pieces * (width / 4);
    if ((threads + 255) / 256 > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "concat grid too large");
    const ConcatPieces p{{in[0], pieces > 1 ? in[1] : in[0], pieces > 2 ? in[2] : in[0], pieces > 3 ? in[3] : in[0]}};
    hipLaunchKernelGGL(herm_concat_bf16_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
                       as_stream(stream), p, pieces, rows, width, static_cast<bf16*>(output));
    return check_launch("koemi_herm_concat_bf16");
}
