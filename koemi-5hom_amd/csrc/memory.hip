// Salient-memory ring update for gfx950.
//
// Reference: model/memory.py:431-455 (LocalKeyValueMemory.salient_tail): the
// carried ring entries followed by the window's entries, ranked by
// (valid ? temporal index : -1), the top `capacity` kept in ascending time
// order, invalid slots zeroed.
//
// One workgroup per batch row. Every position i of the N = S + L entries needs
// the number of valid and of invalid entries after it; a block-wide prefix of
// the per-thread valid counts gives both. With m = min(#valid, capacity) a
// valid entry is kept when fewer than m valid entries follow it, an invalid one
// when fewer than capacity - m invalid entries follow it (the latest invalid
// entries are the filler), and its output slot is capacity - 1 minus the number
// of kept entries after it. The slot -> entry map is built in LDS, then the
// workgroup copies the kept rows (zero rows for invalid slots).
#include "common.hpp"

#include <cstring>
#include <type_traits>

namespace koemi {
namespace {

constexpr int kTailThreads = 256;
constexpr int64_t kMaxCapacity = 4096;
constexpr int kTailSlotsPerBlock = 4;  // output slots copied by one workgroup

// One ring row (keys and values, D entries): copied, widened from KT to T, or
// zeros. VEC: 4 entries per access.
template <typename T, typename KT, bool VEC>
__device__ __forceinline__ void copy_row(const KT* ks, const KT* vs, T* kd, T* vd, int64_t D, bool zero, int tid) {
    if constexpr (VEC && std::is_same<T, KT>::value) {
        using V = typename std::conditional<sizeof(T) == 4, float4, uint2>::type;
        V z;
        memset(&z, 0, sizeof z);
        for (int64_t q = tid; q < D / 4; q += kTailThreads) {
            reinterpret_cast<V*>(kd)[q] = zero ? z : reinterpret_cast<const V*>(ks)[q];
            reinterpret_cast<V*>(vd)[q] = zero ? z : reinterpret_cast<const V*>(vs)[q];
        }
    } else if constexpr (VEC) {
        static_assert(std::is_same<T, float>::value && std::is_same<KT, bf16>::value, "bf16 entries into fp32 rings");
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int64_t q = tid; q < D / 4; q += kTailThreads) {
            reinterpret_cast<float4*>(kd)[q] = zero ? z : load4(ks + 4 * q);
            reinterpret_cast<float4*>(vd)[q] = zero ? z : load4(vs + 4 * q);
        }
    } else {
        for (int64_t d = tid; d < D; d += kTailThreads) {
            kd[d] = zero ? static_cast<T>(0.0f) : static_cast<T>(to_f32(ks[d]));
            vd[d] = zero ? static_cast<T>(0.0f) : static_cast<T>(to_f32(vs[d]));
        }
    }
}

// One workgroup per (ring row, group of kTailSlotsPerBlock output slots):
// every workgroup of a row repeats the (cheap) slot selection in LDS, then
// copies its own slots' key and value rows. VEC: width % 4 == 0 and 16-byte
// (fp32) or 8-byte (half) aligned rows, copied four elements at a time.
//
// Ring rows: blockIdx.x = b * R + r. Row r selects over the carried entries
// and the first Lr = L - (R - 1 - r) * W positions of batch row b, i.e. the
// ring as it stands before position Lr; R = 1 is the ring after all L
// positions (salient_tail), R = L / W + 1 the rings carried into each window
// of W positions plus the final one. TAIL: the last C entries whatever their
// flags (LocalKeyValueMemory.tail, memory.py:385-403), rows copied as stored;
// otherwise the salient rule above (flag = admission).
// Outputs: ring row r < R - 1 of batch row b goes to row b * (R - 1) + r of
// (ok, ov, ovalid), row R - 1 to row b of (fk, fv, fvalid); with R = 1 every
// ring is a final one.
// The window's entries are rows kstride elements apart of type KT (the ring's
// T, or bf16 columns of a wider projection read in place); with wvalid, a
// window entry whose wvalid byte is 0 is copied as zeros (the masking of the
// keys and values of invalid positions, network.py:337-340, done on the way).
template <typename T, typename KT, bool VEC, bool TAIL>
__global__ __launch_bounds__(kTailThreads) void salient_tail_kernel(
    const T* __restrict__ ck, const T* __restrict__ cv, const uint8_t* __restrict__ cvalid, const KT* __restrict__ k,
    const KT* __restrict__ v, int64_t kstride, const uint8_t* __restrict__ wvalid, const uint8_t* __restrict__ adm,
    T* __restrict__ ok, T* __restrict__ ov, uint8_t* __restrict__ ovalid, T* __restrict__ fk, T* __restrict__ fv,
    uint8_t* __restrict__ fvalid, int64_t S, int64_t L, int64_t D, int64_t C, int64_t R, int64_t W) {
    __shared__ int32_t slot_entry[kMaxCapacity];
    __shared__ uint8_t slot_valid[kMaxCapacity];
    __shared__ int64_t wave_tot[kTailThreads / kWave];
    const int64_t b = static_cast<int64_t>(blockIdx.x) / R;
    const int64_t r_in = static_cast<int64_t>(blockIdx.x) - b * R;
    const int64_t Lr = L - (R - 1 - r_in) * W;
    const bool final_ring = r_in == R - 1;
    const int64_t row = final_ring ? b : b * (R - 1) + r_in;
    if (final_ring) {
        ok = fk;
        ov = fv;
        ovalid = fvalid;
    }
    const int tid = threadIdx.x;
    const int64_t N = S + Lr;
    const bool concat = N <= C;
    const int64_t slots = concat ? N : C;
    auto valid_at = [&](int64_t i) -> bool { return i < S ? cvalid[b * S + i] != 0 : adm[b * L + (i - S)] != 0; };
    if (TAIL && !concat) {
        for (int64_t s = tid; s < C; s += kTailThreads) {
            const int64_t i = N - C + s;
            slot_entry[s] = static_cast<int32_t>(i);
            slot_valid[s] = valid_at(i) ? 1 : 0;
        }
    } else if (concat) {
        for (int64_t i = tid; i < N; i += kTailThreads) {
            slot_entry[i] = static_cast<int32_t>(i);
            slot_valid[i] = valid_at(i) ? 1 : 0;
        }
    } else {
        // Contiguous span of positions per thread.
        const int64_t per = (N + kTailThreads - 1) / kTailThreads;
        const int64_t p0 = min(N, tid * per), p1 = min(N, p0 + per);
        int64_t cnt = 0;
        for (int64_t i = p0; i < p1; ++i) cnt += valid_at(i) ? 1 : 0;
        int64_t total_valid;
        int64_t before = block_exclusive_scan<kTailThreads>(cnt, wave_tot, total_valid);  // valid in [0, p0)
        const int64_t m = min(total_valid, C);
        const int64_t total_invalid = N - total_valid;
        for (int64_t i = p0; i < p1; ++i) {
            const bool val = valid_at(i);
            const int64_t valid_after = total_valid - before - (val ? 1 : 0);
            const int64_t invalid_after = total_invalid - (i - before) - (val ? 0 : 1);
            const bool keep = val ? valid_after < m : invalid_after < C - m;
            if (keep) {
                const int64_t slot = C - 1 - (min(valid_after, m) + min(invalid_after, C - m));
                slot_entry[slot] = static_cast<int32_t>(i);
                slot_valid[slot] = val ? 1 : 0;
            }
            if (val) ++before;
        }
    }
    __syncthreads();
    const int64_t s_begin = static_cast<int64_t>(blockIdx.y) * kTailSlotsPerBlock;
    const int64_t s_end = min(slots, s_begin + kTailSlotsPerBlock);
    if (s_begin + tid < s_end) ovalid[row * slots + s_begin + tid] = slot_valid[s_begin + tid];
    // Copy the kept rows; invalid slots are zero unless the outputs are the plain
    // concatenation or the tail of the entries.
    for (int64_t s = s_begin; s < s_end; ++s) {
        const int64_t i = slot_entry[s];
        const bool carried_entry = i < S;
        const bool zero = (!TAIL && !concat && !slot_valid[s]) ||
                          (!carried_entry && wvalid != nullptr && wvalid[b * L + (i - S)] == 0);
        T* kdst = ok + (row * slots + s) * D;
        T* vdst = ov + (row * slots + s) * D;
        if constexpr (std::is_same<T, KT>::value) {
            const T* ksrc = carried_entry ? ck + (b * S + i) * D : k + (b * L + (i - S)) * kstride;
            const T* vsrc = carried_entry ? cv + (b * S + i) * D : v + (b * L + (i - S)) * kstride;
            copy_row<T, T, VEC>(ksrc, vsrc, kdst, vdst, D, zero, tid);
        } else if (carried_entry) {
            copy_row<T, T, VEC>(ck + (b * S + i) * D, cv + (b * S + i) * D, kdst, vdst, D, zero, tid);
        } else {
            // a window entry of another type, widened on the way (bf16 -> fp32 is exact)
            copy_row<T, KT, VEC>(k + (b * L + (i - S)) * kstride, v + (b * L + (i - S)) * kstride, kdst, vdst, D,
                                 zero, tid);
        }
    }
}

// R ring rows per batch row (see salient_tail_kernel); every row has `slots`
// output slots (the windowed form requires S >= C, so that every row has C).
// KT, kstride, wvalid: the window entries' type, row stride and zeroing mask
// (see salient_tail_kernel); KT = T, kstride = D, wvalid = null for stored
// entries.
template <typename T, typename KT = T>
int launch_tail(const void* ck, const void* cv, const uint8_t* cvalid, const void* k, const void* v, const uint8_t* adm,
                void* ok, void* ov, uint8_t* ovalid, void* fk, void* fv, uint8_t* fvalid, int64_t B, int64_t S,
                int64_t L, int64_t D, int64_t C, int64_t R, int64_t W, bool tail, const char* what, hipStream_t s,
                int64_t kstride = -1, const uint8_t* wvalid = nullptr) {
    if (kstride < 0) kstride = D;
    const int64_t slots = S + L <= C ? S + L : C;
    const dim3 grid(static_cast<unsigned>(B * R), static_cast<unsigned>((slots + kTailSlotsPerBlock - 1) / kTailSlotsPerBlock));
    const size_t align = sizeof(T) == 4 ? 16 : 8;
    const size_t kalign = sizeof(KT) == 4 ? 16 : 8;
    auto aligned = [&](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % align == 0; };
    auto kaligned = [&](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % kalign == 0; };
    const bool vec = D % 4 == 0 && aligned(ck) && aligned(cv) && kaligned(k) && kaligned(v) && aligned(ok) &&
                     aligned(ov) && aligned(fk) && aligned(fv) && (kstride * sizeof(KT)) % kalign == 0;
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(kTailThreads), 0, s, static_cast<const T*>(ck), static_cast<const T*>(cv),
                           cvalid, static_cast<const KT*>(k), static_cast<const KT*>(v), kstride, wvalid, adm,
                           static_cast<T*>(ok), static_cast<T*>(ov), ovalid, static_cast<T*>(fk), static_cast<T*>(fv),
                           fvalid, S, L, D, C, R, W);
    };
    if (tail) {
        if (vec) launch(salient_tail_kernel<T, KT, true, true>);
        else launch(salient_tail_kernel<T, KT, false, true>);
    } else {
        if (vec) launch(salient_tail_kernel<T, KT, true, false>);
        else launch(salient_tail_kernel<T, KT, false, false>);
    }
    return check_launch(what);
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" int koemi_salient_tail(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                                  const void* keys, const void* values, const uint8_t* admission, void* out_keys,
                                  void* out_values, uint8_t* out_valid, int64_t batch, int64_t carried, int64_t length,
                                  int64_t width, int64_t capacity, int dtype, koemi_stream_t stream) {
    if (batch < 0 || carried < 0 || length < 0 || width < 1)
        return fail(KOEMI_ERR_INVALID, "salient_tail sizes must be non-negative with a positive width");
    if (capacity < 1 || capacity > kMaxCapacity)
        return fail(KOEMI_ERR_UNSUPPORTED, "salient_tail capacity must be in [1, %lld]", static_cast<long long>(kMaxCapacity));
    if (batch > 0x7fffffffLL || carried + length > 0x7fffffffLL)
        return fail(KOEMI_ERR_UNSUPPORTED, "salient_tail: too many rows or entries");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "salient_tail does not support dtype %s", dtype_name(dtype));
    const int64_t slots = carried + length <= capacity ? carried + length : capacity;
    if (batch == 0 || slots == 0) return KOEMI_OK;
    if ((carried > 0 && (!carried_keys || !carried_values || !carried_valid)) ||
        (length > 0 && (!keys || !values || !admission)) || !out_keys || !out_values || !out_valid)
        return fail(KOEMI_ERR_INVALID, "salient_tail received a null pointer");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case KOEMI_F32:
            return launch_tail<float>(carried_keys, carried_values, carried_valid, keys, values, admission, out_keys,
                                      out_values, out_valid, out_keys, out_values, out_valid, batch, carried, length,
                                      width, capacity, 1, 0, false, "koemi_salient_tail", s);
        case KOEMI_F16:
            return launch_tail<f16>(carried_keys, carried_values, carried_valid, keys, values, admission, out_keys,
                                    out_values, out_valid, out_keys, out_values, out_valid, batch, carried, length,
                                    width, capacity, 1, 0, false, "koemi_salient_tail", s);
        default:
            return launch_tail<bf16>(carried_keys, carried_values, carried_valid, keys, values, admission, out_keys,
                                     out_values, out_valid, out_keys, out_values, out_valid, batch, carried, length,
                                     width, capacity, 1, 0, false, "koemi_salient_tail", s);
    }
}

extern "C" int koemi_window_rings(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                                  const void* keys, const void* values, int key_dtype, int64_t key_row_stride,
                                  const uint8_t* key_valid, const uint8_t* flags, void* out_keys, void* out_values,
                                  uint8_t* out_valid, void* final_keys, void* final_values, uint8_t* final_valid,
                                  int64_t batch, int64_t carried, int64_t length, int64_t window, int64_t width,
                                  int64_t capacity, int tail, int dtype, koemi_stream_t stream) {
    if (batch < 0 || length < 0 || width < 1 || window < 1)
        return fail(KOEMI_ERR_INVALID, "window rings need non-negative sizes, a positive width and window");
    if (length % window) return fail(KOEMI_ERR_INVALID, "window rings need a length that is a multiple of the window");
    // no per-window outputs: the final ring alone (one ring row per batch row)
    const bool final_only = out_keys == nullptr && out_values == nullptr && out_valid == nullptr;
    if (capacity < 1 || capacity > kMaxCapacity || (carried < capacity && !final_only) || carried < 0)
        return fail(KOEMI_ERR_UNSUPPORTED, "window rings need a carried ring at capacity (capacity in [1, %lld])",
                    static_cast<long long>(kMaxCapacity));
    const int64_t rows = final_only ? 1 : length / window + 1;
    if (batch * rows > 0x7fffffffLL || carried + length > 0x7fffffffLL)
        return fail(KOEMI_ERR_UNSUPPORTED, "window rings: too many rows or entries");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "window rings do not support dtype %s", dtype_name(dtype));
    if (batch == 0) return KOEMI_OK;
    if ((carried > 0 && (!carried_keys || !carried_values || !carried_valid)) ||
        (length > 0 && (!keys || !values || !flags)) ||
        (length > 0 && !final_only && (!out_keys || !out_values || !out_valid)) || !final_keys || !final_values ||
        !final_valid)
        return fail(KOEMI_ERR_INVALID, "window rings received a null pointer");
    if (key_row_stride == 0) key_row_stride = width;
    if (key_row_stride < width) return fail(KOEMI_ERR_INVALID, "window rings: key row stride below the width");
    hipStream_t s = as_stream(stream);
    const bool t = tail != 0;
    const int64_t R = rows;
    if (key_dtype != dtype || key_row_stride != width || key_valid != nullptr) {
        // entries read in place (bf16 columns of a projection into fp32 rings)
        if (dtype != KOEMI_F32 || (key_dtype != KOEMI_F32 && key_dtype != KOEMI_BF16))
            return fail(KOEMI_ERR_UNSUPPORTED, "window rings read in place take fp32 rings and fp32 or bf16 entries");
        if (key_dtype == KOEMI_BF16)
            return launch_tail<float, bf16>(carried_keys, carried_values, carried_valid, keys, values, flags, out_keys,
                                            out_values, out_valid, final_keys, final_values, final_valid, batch,
                                            carried, length, width, capacity, R, window, t, "koemi_window_rings", s,
                                            key_row_stride, key_valid);
        return launch_tail<float, float>(carried_keys, carried_values, carried_valid, keys, values, flags, out_keys,
                                         out_values, out_valid, final_keys, final_values, final_valid, batch, carried,
                                         length, width, capacity, R, window, t, "koemi_window_rings", s, key_row_stride,
                                         key_valid);
    }
    switch (dtype) {
        case KOEMI_F32:
            return launch_tail<float>(carried_keys, carried_values, carried_valid, keys, values, flags, out_keys,
                                      out_values, out_valid, final_keys, final_values, final_valid, batch, carried,
                                      length, width, capacity, rows, window, t, "koemi_window_rings", s);
        case KOEMI_F16:
            return launch_tail<f16>(carried_keys, carried_values, carried_valid, keys, values, flags, out_keys,
                                    out_values, out_valid, final_keys, final_values, final_valid, batch, carried,
                                    length, width, capacity, rows, window, t, "koemi_window_rings", s);
        default:
            return launch_tail<bf16>(carried_keys, carried_values, carried_valid, keys, values, flags, out_keys,
                                     out_values, out_valid, final_keys, final_values, final_valid, batch, carried,
                                     length, width, capacity, rows, window, t, "koemi_window_rings", s);
    }
}
