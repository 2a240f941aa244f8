// The bf16 MFMA main loop shared by the grouped expert GEMM and the gate
// projection + scan: a 256 x BNT block tile, four waves in 2 x 2, each owning
// 128 rows x BNT / 2 columns of it as 4 x NT tiles of v_mfma_f32_32x32x16_bf16
// (fp32 accumulators). K advances in 32-wide steps through a ring of LDS
// stages (A rows then B rows, 64 bytes per row) filled by
// global_load_lds_dwordx4, which writes each lane's 16 bytes straight into LDS
// at M0 + 16 * lane without passing through registers. A stage row is four
// 16-byte K groups; group g of row r sits at slot g ^ ((r >> 2) & 3), so the
// sixteen rows read by any sixteen consecutive lanes fill 256 distinct bytes
// of banks (conflict-free 16-byte fragment reads).
#pragma once

#include "common.hpp"

#include <type_traits>

namespace koemi {
namespace mfma_stage {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kBM = 256;                               // block tile rows (A)
constexpr int kBK = 32;                                // K per stage
constexpr int kThreads = 256;                          // four waves
constexpr uint32_t kOperandBytes = kBM * kBK * 2u;     // the A operand of one stage (bf16)

// Byte offset of K group g (16 bytes) of row r inside one operand stage.
__device__ __forceinline__ int slot_swizzle(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ uint32_t stage_slot(int r, int g) {
    return static_cast<uint32_t>(r * (kBK * 2) + ((g ^ slot_swizzle(r)) << 4));
}

// Asynchronous 16-byte-per-lane copy global -> LDS (lane l writes M0 + 16 l).
// Issued through inline assembly so that the compiler does not order every
// later LDS read after it (it cannot tell the ring stages apart); completion is
// tracked explicitly with vmcnt, and ordering against other waves' reads of the
// stage comes from the barrier (volatile asm is never reordered against other
// volatile asm). M0 is restored afterwards.
// The source is a wave-uniform 64-bit base (SGPRs) plus a per-lane 32-bit byte
// offset, so issuing a copy costs no vector instructions.
__device__ __forceinline__ void lds_dma16(uint32_t lds_byte_addr, const void* base, uint32_t byte_off) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %2, %3\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds_byte_addr), "v"(byte_off), "s"(base));
}

__device__ __forceinline__ const void* uniform_ptr(const void* p) {
    const uint64_t u = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Waits until at most n tiles of this wave's stage copies are outstanding
// (CPT copies per tile and wave: eight for 256-wide tiles, six for 128-wide),
// then joins the workgroup.
template <int CPT>
__device__ __forceinline__ void wait_tiles_and_sync(int64_t n) {
    static_assert(CPT == 8 || CPT == 6, "stage copies per tile");
    if (CPT == 8) {
        if (n >= 3) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
        else if (n == 2) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else if (n == 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
        if (n >= 1) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Tile geometry of a 256 x BNT block tile.
template <int BNT>
struct TileShape {
    static constexpr int kNT = BNT / 64;                                 // n-tiles (32 wide) per wave
    static constexpr int kStages = BNT == 256 ? 4 : 3;
    static constexpr uint32_t kStageBytes = static_cast<uint32_t>(kBM + BNT) * kBK * 2u;
    static constexpr int kCopies = 4 + kNT;                              // 1 KiB stage copies per wave and tile
    static constexpr int kWgPerCu = BNT == 256 ? 1 : 2;
    static constexpr int64_t kPartialFloats = static_cast<int64_t>(kBM) * BNT;
};

// The K loop of one block tile: nk (>= 2) K steps of the A rows at a_base +
// a_off[i] and the B rows at b_base + b_off[i] (byte offsets of this lane's
// 16-byte piece of its stage copies, relative to K step 0) into acc[m-tile][
// n-tile] (zeroed by the caller). a_lds / b_lds: this wave's copy
// destinations in stage 0; a_row / b_row: the stage rows of the wave's
// fragments. WEIGHTS_FIRST: the B fragment is the MFMA's first operand, so a
// lane's accumulators are four consecutive B columns of one A row (element v of
// lane l: A row l % 32, B column 8 (v / 4) + 4 (l / 32) + v % 4); otherwise
// one B column of sixteen A rows (element v of lane l: B column l % 32, A row
// 8 (v / 4) + 4 (l / 32) + v % 4).
//
// The prologue issues K tiles 0 .. kStages - 2; step kt issues the copy of K
// tile kt + kStages - 1 (while there is one) into the stage consumed by step
// kt - 1, so up to kStages - 3 tiles are in flight behind the one waited for at
// every barrier; no copy is issued past the last tile, so none is outstanding
// when the loop returns. Each MFMA is followed by memory instructions for later
// work (stage copies and fragment reads), pinned in place by scheduling
// barriers, so that they issue while the matrix pipe is busy instead of in a
// burst that leaves it idle. 256-wide tiles: 16 MFMAs per half step, a copy
// after every fourth one in both halves (eight per step, evenly spaced: the
// copies of a step land in the stage of tile kt - 1, free for the whole step)
// and a fragment read after every odd one. 128-wide: 8 MFMAs per half step,
// copy j after MFMA j (six) and fragment j - 2 after MFMA j >= 2.
template <int BNT, bool WEIGHTS_FIRST>
__device__ __forceinline__ void stage_loop(char* lds, const bf16* a_base, const bf16* b_base,
                                           const uint32_t (&a_off)[4], const uint32_t (&b_off)[BNT / 64],
                                           uint32_t a_lds, uint32_t b_lds, const int (&a_row)[4],
                                           const int (&b_row)[BNT / 64], int64_t nk,
                                           f32x16 (&acc)[4][BNT / 64]) {
    using TS = TileShape<BNT>;
    constexpr int NT = TS::kNT;
    constexpr int kStages = TS::kStages;
    constexpr uint32_t kStageBytes = TS::kStageBytes;
    constexpr int CPT = TS::kCopies;
    const int lane = lane_id();
    const int fg = lane >> 5;

    // Copy i of a stage: i < 4 is A chunk i of this wave, i >= 4 B chunk i - 4.
    auto issue_one = [&](int64_t kt, int stage, int i) {
        if (i < 4)
            lds_dma16(a_lds + stage * kStageBytes + i * 1024, a_base + kt * kBK, a_off[i]);
        else
            lds_dma16(b_lds + stage * kStageBytes + (i - 4) * 1024, b_base + kt * kBK, b_off[i - 4]);
    };
    auto issue = [&](int64_t kt, int stage) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) issue_one(kt, stage, i);
    };
    auto read_frags = [&](int64_t kt, int kk, bf16x8 (&af)[4], bf16x8 (&bfr)[NT]) {
        const char* As = lds + (kt % kStages) * kStageBytes;
        const char* Bs = As + kOperandBytes;
#pragma unroll
        for (int t = 0; t < 4; ++t) af[t] = *reinterpret_cast<const bf16x8*>(As + stage_slot(a_row[t], kk * 2 + fg));
#pragma unroll
        for (int t = 0; t < NT; ++t) bfr[t] = *reinterpret_cast<const bf16x8*>(Bs + stage_slot(b_row[t], kk * 2 + fg));
    };
    // Fragment f of a K step (4 + NT of them), in the order the MFMAs of the
    // step consume them: A m-tile 0, B n-tiles 0 .. NT - 1, A m-tiles 1-3.
    auto read_frag = [&](int64_t kt, int kk, int f, bf16x8 (&af)[4], bf16x8 (&bfr)[NT]) {
        const char* As = lds + (kt % kStages) * kStageBytes;
        if (f >= 1 && f <= NT)
            bfr[f - 1] = *reinterpret_cast<const bf16x8*>(As + kOperandBytes + stage_slot(b_row[f - 1], kk * 2 + fg));
        else {
            const int t = f == 0 ? 0 : f - NT;
            af[t] = *reinterpret_cast<const bf16x8*>(As + stage_slot(a_row[t], kk * 2 + fg));
        }
    };
    auto mfma_one = [&](int j, const bf16x8 (&af)[4], const bf16x8 (&bfr)[NT]) {
        if constexpr (WEIGHTS_FIRST)
            acc[j / NT][j % NT] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j % NT], af[j / NT], acc[j / NT][j % NT], 0, 0, 0);
        else
            acc[j / NT][j % NT] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[j / NT], bfr[j % NT], acc[j / NT][j % NT], 0, 0, 0);
    };

#pragma unroll
    for (int i = 0; i < kStages - 1; ++i)
        if (i < nk) issue(i, i);
    wait_tiles_and_sync<CPT>(min(nk, static_cast<int64_t>(kStages - 1)) - 1);
    bf16x8 a0[4], b0[NT], a1[4], b1[NT];
    read_frags(0, 0, a0, b0);
    constexpr int MK = 4 * NT;  // MFMAs per half step
    auto k_step = [&](int64_t kt, auto copy_tag) {
        constexpr bool kCopy = decltype(copy_tag)::value;
        // Tile kt + 1 has landed for every wave (later copies may still be in
        // flight: tiles kt + 2 .. min(kt + kStages - 2, nk - 1)), and every
        // wave is done with the stage of tile kt - 1, which this step's copy
        // overwrites.
        if (kCopy) wait_tiles_and_sync<CPT>(kStages - 3);
        else wait_tiles_and_sync<CPT>(max(min(nk - 2 - kt, static_cast<int64_t>(kStages - 3)), int64_t(0)));
        const int sc = static_cast<int>((kt + kStages - 1) % kStages);
#pragma unroll
        for (int j = 0; j < MK; ++j) {
            mfma_one(j, a0, b0);
            if constexpr (NT == 4) {
                if (j % 2 == 0) {
                    if constexpr (kCopy) {
                        if (j % 4 == 0) issue_one(kt + kStages - 1, sc, j / 4);
                    }
                } else {
                    read_frag(kt, 1, j / 2, a1, b1);
                }
            } else {
                if constexpr (kCopy) {
                    if (j < CPT) issue_one(kt + kStages - 1, sc, j);
                }
                if (j >= 2) read_frag(kt, 1, j - 2, a1, b1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        const int64_t kn = min(kt + 1, nk - 1);  // the last step re-reads its own stage harmlessly
#pragma unroll
        for (int j = 0; j < MK; ++j) {
            mfma_one(j, a1, b1);
            if constexpr (NT == 4) {
                if constexpr (kCopy) {
                    if (j % 4 == 0) issue_one(kt + kStages - 1, sc, 4 + j / 4);
                }
                if (j % 2 == 1) read_frag(kn, 0, j / 2, a0, b0);
            } else {
                if (j >= 2) read_frag(kn, 0, j - 2, a0, b0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    int64_t kt = 0;
    for (; kt + kStages - 1 < nk; ++kt) k_step(kt, std::true_type{});
    for (; kt < nk; ++kt) k_step(kt, std::false_type{});
}

}  // namespace mfma_stage
}  // namespace koemi
