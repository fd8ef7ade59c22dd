// gemm16_kernel.h — f16 MFMA contraction for gfx950 with direct global->LDS loads (no register staging).
//
// Block tile BM x BN (256x256 or 128x128) shared by WVM x WVN wave64s, K in LDS stages of 32 or 64
// halves with NS stages in flight.
// Every operand tile is fetched with global_load_lds_dwordx4 (each lane's 16 bytes land at
// LDS base + 16*lane), so loads for later stages are in flight while stage k is contracted, and no
// VGPRs or ds_write instructions are spent on staging. The layouts are chosen so that the fetch order
// produces a bank-conflict-free LDS image (the LDS of gfx950 has 64 four-byte banks):
//   K-contiguous operand ([rows][K]): rows of 64 or 128 bytes are packed into 256-byte super-rows
//     whose 16-byte slots are XOR-swizzled by the super-row index; fragments are ds_read_b128.
//   MN-contiguous operand ([K][rows]): k-rows stay in the stored orientation, 32-byte segments
//     XOR-swizzled by 2*(k & 3); fragments are read with two ds_read_b64_tr_b16, the CDNA4 LDS
//     transpose read (within 16 lanes, lane j addressing T[kb + j/4][mb + 4*(j%4)] receives
//     T[kb..kb+3][mb + j]), so transposed operands cost no extra pass and no register shuffles.
// Fragments of k-step s+1 are read while the MFMAs of k-step s run. Accumulation is f32
// (codegen/lower.go:667-716 accumulates f16 reduces in f32); f16 products are exact in f32.
// Each variant (a parameter set of the template, table Var<V> at the end) is instantiated in its own
// translation unit (gemm16_var.hip) so that the variants compile in parallel.
#pragma once
#include <type_traits>
#include "ah_common.h"
#include "gemm.h"
#include "gemm_epi.h"

namespace ah {
namespace g16 {

typedef half_t h8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;

// Byte offset of (row r, 16-byte chunk c) in a K-contiguous tile whose rows hold BK halves:
// 256-byte super-rows of 256/(2*BK) rows, 16-byte slots XOR-swizzled by the super-row index.
template <int BK>
__device__ __forceinline__ int koff(int r, int c) {
    constexpr int CH = BK / 8, SR = 16 / CH;        // chunks per row, rows per super-row
    const int q = r / SR;
    return q * 256 + ((((r % SR) * CH + c) ^ (q & 15)) << 4);
}

// Byte offset of element (k-row k, column m) in an MN-contiguous tile of R columns: 32-byte segments
// XOR-swizzled by 2*(k & 3) + ((k >> 3) & 1). The first term spreads the four k-rows one transposing
// read covers over the banks; the second separates k-rows 8 apart, which the 16x16 fragments' lane
// groups read together.
__device__ __forceinline__ int mn_swz(int k) { return ((k & 3) << 1) ^ ((k >> 3) & 1); }
template <int R>
__device__ __forceinline__ int mnoff(int k, int m) {
    return k * (R * 2) + (((m >> 4) ^ mn_swz(k)) << 5) + ((m & 15) << 1);
}

// One 16-byte-per-lane global->LDS DMA issued from inline asm: the compiler's wait-count model does
// not see it, so it adds no conservative waits (an LDS-DMA the compiler knows about makes it wait
// for every outstanding LDS read at the next use of any of them). The kernel orders these loads
// with its own explicit s_waitcnt vmcnt. M0 (the DMA's LDS base) is written here; the compiler
// reserves M0 and warns about the clobber, but no instruction it emits in these kernels reads M0 (no
// builtin LDS-DMA, no dynamic register indexing on the fetch-mode-3 path), so nothing is disturbed.
// The global address is a wave-uniform base in SGPRs plus a 32-bit per-lane offset (the saddr form),
// and the LDS destination a wave-uniform 32-bit LDS address, so a DMA costs no VALU address work.
__device__ __forceinline__ void dma16(uint32_t voff, const char *sbase, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
                 : "memory", "m0");
}

// Workgroup barrier for the stage pipeline: waits for this wave's LDS reads only. (__syncthreads()
// is a release fence as well, which makes the wave wait for every outstanding global->LDS load,
// including the stages still meant to be in flight.) Stage data is complete once every wave has
// passed its own s_waitcnt vmcnt for that stage and this barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// L2 prefetch of one 128-byte line: a 4-byte-per-lane LDS-DMA into a junk LDS slot that nothing
// reads (a load into a VGPR would need that register reserved against the load's late write-back).
__device__ __forceinline__ void prefetch_line(const char *g, const char *junk) {
    const uint32_t l = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)junk;
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(l))
                 : "memory", "m0");
}

// Per-lane global byte offsets for the 1 KiB blocks this wave fetches (stage-independent part).
template <int R, int T, int BK, int NW>
struct Fetch {
    static constexpr int NB = R * BK * 2 / 1024;   // 1 KiB blocks per tile
    static constexpr int PER = NB / NW;            // blocks per wave
    static_assert(PER * NW == NB, "tile blocks must split evenly over the waves");
    uint32_t off[PER];
    __device__ __forceinline__ void init(long ld, int r0, int rmax, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int b = wave * PER + j;
            if constexpr (T == 0) {
                constexpr int CH = BK / 8, SR = 16 / CH;
                const int q = 4 * b + (lane >> 4);
                const int x = (lane & 15) ^ (q & 15);
                const int row = min(r0 + q * SR + x / CH, rmax - 1);
                off[j] = (uint32_t)(((long)row * ld + (x % CH) * 8) * 2);
            } else {
                constexpr int ROWS = 512 / R;                 // k-rows per block
                const int kk = b * ROWS + (16 * lane) / (2 * R);
                const int pos16 = ((16 * lane) % (2 * R)) / 16;
                const int seg = (pos16 >> 1) ^ mn_swz(kk);
                const int m = min(r0 + seg * 16 + (pos16 & 1) * 8, rmax - 8);
                off[j] = (uint32_t)(((long)kk * ld + m) * 2);
            }
        }
    }
    // Issue this wave's loads of the stage starting at k0 into `tile` (a 1 KiB-aligned LDS region).
    __device__ __forceinline__ void issue(const char *base, long ld, int k0, char *tile, int wave) const {
#pragma unroll
        for (int j = 0; j < PER; j++) issue_one(j, base, ld, k0, tile, wave);
    }
    __device__ __forceinline__ void issue_one(int j, const char *base, long ld, int k0, char *tile, int wave) const {
        const long adv = T == 0 ? (long)k0 * 2 : (long)k0 * ld * 2;
        __builtin_amdgcn_global_load_lds((const void *)(base + adv + off[j]), (void *)(tile + (wave * PER + j) * 1024),
                                         16, 0, 0);
    }
    // asm DMAs: tile_lds is the tile's 32-bit LDS address and wave is wave-uniform (an SGPR)
    __device__ __forceinline__ void issue_one_asm(int j, const char *base, long ld, int k0, uint32_t tile_lds, int wave) const {
        const long adv = T == 0 ? (long)k0 * 2 : (long)k0 * ld * 2;
        dma16(off[j], base + adv, tile_lds + (uint32_t)((wave * PER + j) * 1024));
    }
    __device__ __forceinline__ void issue_asm(const char *base, long ld, int k0, uint32_t tile_lds, int wave) const {
#pragma unroll
        for (int j = 0; j < PER; j++) issue_one_asm(j, base, ld, k0, tile_lds, wave);
    }
};

// L2 prefetch of one operand's stage (k = k0 .. k0+63): the stage is R lines of 128 bytes (a
// K-contiguous row holds 64 halves = one line; an MN-contiguous k-row of R halves holds R/64 lines).
// Line i of the stage is touched by thread i (callers pass i < R, ragged rows clamped).
template <int R, int T>
__device__ __forceinline__ void prefetch_stage(const char *base, long ld, int r0, int rmax, int k0, int i,
                                               const char *junk) {
    if constexpr (T == 0) {
        const int row = min(r0 + i, rmax - 1);
        prefetch_line(base + ((long)row * ld + k0) * 2, junk);
    } else {
        constexpr int LPR = R / 64;
        const int col = min(r0 + (i % LPR) * 64, rmax - 1);
        prefetch_line(base + ((long)(k0 + i / LPR) * ld + col) * 2, junk);
    }
}

template <int R, int T, int BK>
__device__ __forceinline__ h8 frag(const char *tile, int r, int s, int lane) {
    if constexpr (T == 0) {
        return *(const h8 *)(tile + koff<BK>(r + (lane & 31), 2 * s + (lane >> 5)));
    } else {
        const int g = lane >> 4, j = lane & 15;
        const int m = r + 16 * (g & 1) + 4 * (j & 3);
        const int k = 16 * s + 8 * (g >> 1) + (j >> 2);
        s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)(tile + mnoff<R>(k, m)));
        s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)(tile + mnoff<R>(k + 4, m)));
        typedef short s8 __attribute__((ext_vector_type(8)));
        s8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        return __builtin_bit_cast(h8, v);
    }
}

// Fragment of a 16x16x32 MFMA: lane l holds rows r + l%16, k = 32*s + 8*(l/16) .. +7 (the same
// eight-halves-per-lane form as frag, over 16 rows and 32 k).
template <int R, int T, int BK>
__device__ __forceinline__ h8 frag16(const char *tile, int r, int s, int lane) {
    if constexpr (T == 0) {
        return *(const h8 *)(tile + koff<BK>(r + (lane & 15), 4 * s + (lane >> 4)));
    } else {
        const int g = lane >> 4, j = lane & 15;
        const int m = r + 4 * (j & 3);
        const int k = 32 * s + 8 * g + (j >> 2);
        s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)(tile + mnoff<R>(k, m)));
        s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)(tile + mnoff<R>(k + 4, m)));
        typedef short s8 __attribute__((ext_vector_type(8)));
        s8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        return __builtin_bit_cast(h8, v);
    }
}

// VEPI: every wave tile is in bounds and the epilogue arrays admit vector access, so the LDS-staged
// vector epilogue is used (chosen on the host; a kernel holding both epilogues spills registers).
// BK: k per LDS stage (32 or 64); NS: LDS stages in flight (the fetch of stage k+NS-1 is issued
// while stage k is contracted). WVM x WVN waves share the tile: with 2x2 each wave holds a 128x128
// accumulator (one wave per SIMD); with 4x2 on a 256x256 tile each wave holds 64x128 and two waves
// share a SIMD, so one wave's MFMAs cover the other's LDS reads and barrier waits.
// FETCH: where a stage's global->LDS fetches are issued. 0: as one group after the first k-step's
// fragment reads; 1: spread between the MFMAs; 2: as one group right after the stage barrier, before
// any fragment read. (An LDS-DMA issue makes the compiler wait for every outstanding LDS read at the
// next MFMA, so with 0 and 1 the fragment reads of k-step s+1 are waited on before the MFMAs of s.)
// 3: like 2, but the DMAs are issued from inline asm (no compiler-inserted waits) and every thread
// also prefetches one line of stage kt+NS into L2, so the DMA of that stage one iteration later hits
// L2 instead of waiting on the Infinity Cache or HBM. Needs k=64 stages and 2*BM threads.
// 4: like 3 without the L2 prefetch (any stage depth).
// 5: asm DMAs as in 4, but interleaved one per MFMA (or per few MFMAs) through the k-step that follows
//    the stage barrier, so that a wave never stalls its MFMA issue behind a burst of vector-memory
//    instructions (needs XB; the k-step after the barrier is the last one of the previous stage).
// 6: like 5, and in the other k-steps the fragment reads of k-step s+1 are placed one (or a few)
//    per MFMA at the start of k-step s (scheduling-group barriers), leaving the last MFMAs of the
//    k-step to cover the read latency instead of letting reads cluster at its end.
// 7: like 6, with the fragment reads spread evenly over the whole k-step (one every NM/NR MFMAs).
// XB: cross-barrier fragment prefetch (fetch modes 2-4). The wait and barrier for stage k+1 move in
// front of the last k-step of stage k, so the first fragment reads of stage k+1 are in flight during
// the last MFMAs of stage k instead of being exposed after the barrier.
// KG: k-groups. With KG = 2 the workgroup holds two sets of WVM x WVN waves on the same tile; group g
// contracts the g-th half of K through its own LDS stages; at the end the groups exchange halves of
// their accumulators through LDS, and each adds and finishes one half of the tile. Two waves then
// share each SIMD on tiles whose accumulators leave room for only one wave set (the 128x128 tile).
// LDS bytes of a variant's tile program (operand stages, epilogue staging, k-group reduction).
template <int BM, int BN, int BK, int NS, int WVM, int WVN, int FETCH, int KG>
struct G16Smem {
    static constexpr int NW = WVM * WVN, WM = BM / WVM;
    static constexpr int STAGE = BM * BK * 2 + BN * BK * 2;
    static constexpr int SMEM0 = (NS * STAGE > NW * WM * 256) ? NS * STAGE : NW * WM * 256;
    static constexpr int SMEMG = FETCH == 3 ? SMEM0 + NW * 256 : SMEM0;   // + per-wave prefetch junk slots
    static constexpr int SMEMR = KG > 1 ? BM * BN * 4 : 0;                // k-group reduction buffer
    static constexpr int SMEM = KG * SMEMG > SMEMR ? KG * SMEMG : SMEMR;
};

// Hook between a tile's main loop and its epilogue (single-k-group variants): run() may replace the
// accumulators (e.g. with the sum of a K split's partials) and returns false when this workgroup is
// not to run the epilogue. G16NoFold is the plain tile.
struct G16NoFold {
    template <int FM, int FN, int NT>
    __device__ __forceinline__ bool run(floatx16 (&)[FM][FN], int) const { return true; }
};

// Tile origin of tile index L of a tiles_m x tiles_n grid: tile rows in groups of 4, walked
// column-major within a group, so that concurrent tiles share operand panels in L2.
__device__ __forceinline__ void g16_tile_origin(int L, int tiles_m, int tiles_n, int BM, int BN, int &m0, int &n0) {
    constexpr int G = 4;
    const int group = L / (G * tiles_n);
    const int gm0 = group * G;
    const int gsz = min(G, tiles_m - gm0);
    const int rem = L - group * G * tiles_n;
    m0 = (gm0 + rem % gsz) * BM;
    n0 = (rem / gsz) * BN;
}

// One output tile at (m0, n0) over k in [kbase, kbase + klen), then fold.run (single k-group) and
// the epilogue. smem holds G16Smem<...>::SMEM bytes.
template <int BM, int BN, int TA, int TB, int EPI, bool VEPI, int BK, int NS, int WVM, int WVN, int FETCH, bool XB, int KG,
          class Fold, bool HL = false, int MI = 32>
__device__ __forceinline__ void g16_tile(const GemmDesc &d, char *smem, int m0, int n0, long kbase, int klen,
                                         const Fold &fold) {
    using SM = G16Smem<BM, BN, BK, NS, WVM, WVN, FETCH, KG>;
    constexpr int NW = WVM * WVN;
    constexpr int WM = BM / WVM, WN = BN / WVN, FM = WM / 32, FN = WN / 32;
    constexpr int ABYTES = BM * BK * 2, STAGE = SM::STAGE;
    // MI: the MFMA shape, 32 (32x32x16) or 16 (16x16x32). A k-step is one MFMA's k; fragments are
    // 32 or 16 rows, FA of A and FB of B per k-step, FA*FB MFMAs per k-step.
    static_assert(MI == 32 || MI == 16, "MFMA shape 32x32x16 or 16x16x32");
    constexpr int KS = MI == 32 ? BK / 16 : BK / 32;                      // MFMA k-steps per stage
    constexpr int FA = MI == 32 ? FM : 2 * FM, FB = MI == 32 ? FN : 2 * FN;
    static_assert(!XB || KS % 2 == 0, "cross-barrier prefetch opens the next stage in fragment slot 0");
    static_assert(VEPI || MI == 32, "MI 16 tiles use the LDS-staged epilogue");
    constexpr int PERSTAGE = Fetch<BM, TA, BK, NW>::PER + Fetch<BN, TB, BK, NW>::PER;
    constexpr int SMEM0 = SM::SMEM0, SMEMG = SM::SMEMG;
    static_assert(WN % 64 == 0, "the LDS epilogue works in 64-column slabs");
    static_assert(!XB || FETCH >= 2, "cross-barrier prefetch needs the fetches grouped at the barrier");
    static_assert(FETCH < 5 || XB, "fetch modes 5-7 interleave the fetches with the k-step after the barrier (XB)");

    const int lane = threadIdx.x & 63;
    const int kg = KG > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) / NW : 0;   // k-group
    const int tid = threadIdx.x - kg * 64 * NW, wave = tid >> 6;                             // within the group
    const int wm0 = (wave / WVN) * WM, wn0 = (wave % WVN) * WN;
    char *gsm = smem + kg * SMEMG;                                                          // the group's LDS
    // the same region as a 32-bit LDS address, and the wave index as a wave-uniform value, for the asm DMAs
    const uint32_t gsm_lds = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)smem + kg * SMEMG;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);

    Fetch<BM, TA, BK, NW> fa;
    Fetch<BN, TB, BK, NW> fb;
    fa.init(d.lda, m0, d.M, wave, lane);
    fb.init(d.ldb, n0, d.N, wave, lane);
    const char *Ab = (const char *)d.A, *Bb = (const char *)d.B;
    const int nk = klen / BK / KG;
    // HL (two-plane A, GemmDesc::A2): the stages run over the group's part of K twice, the second time
    // from A2. Stage offsets k >= nk*BK address A2 and B through bases moved back by one pass, so every
    // fetch keeps its (base, k) form.
    const char *Ab2v = nullptr, *Bbv = nullptr;
    {   // this group's part of K starts at kbase + kg * nk * BK
        const long k0 = kbase + (long)kg * nk * BK;
        Ab += TA == 0 ? k0 * 2 : k0 * d.lda * 2;
        Bb += TB == 0 ? k0 * 2 : k0 * d.ldb * 2;
        if constexpr (HL) {
            const long span = (long)nk * BK;
            Ab2v = (const char *)d.A2 + (TA == 0 ? (k0 - span) * 2 : (k0 - span) * d.lda * 2);
            Bbv = Bb - (TB == 0 ? span * 2 : span * d.ldb * 2);
        }
    }
    const int nkt = HL ? 2 * nk : nk;   // stages of the loop
    auto ab = [&](int k) -> const char * {
        if constexpr (HL) return k >= nk * BK ? Ab2v : Ab;
        else return Ab;
    };
    auto bb = [&](int k) -> const char * {
        if constexpr (HL) return k >= nk * BK ? Bbv : Bb;
        else return Bb;
    };

    // 32x32 accumulator blocks (MI 32) or 16x16 ones (MI 16); the epilogue reads either through
    // AccView as FM x FN 32x32 blocks
    floatx16 acc[MI == 32 ? FM : 1][MI == 32 ? FN : 1];
    floatx4 acc4[MI == 16 ? FA : 1][MI == 16 ? FB : 1];
    if constexpr (MI == 32) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[i][j] = (floatx16){};
    } else {
#pragma unroll
        for (int i = 0; i < FA; i++)
#pragma unroll
            for (int j = 0; j < FB; j++) acc4[i][j] = (floatx4){};
    }
    auto fragA = [&](const char *t, int i, int ks) -> h8 {
        if constexpr (MI == 32) return frag<BM, TA, BK>(t, wm0 + i * 32, ks, lane);
        else return frag16<BM, TA, BK>(t, wm0 + i * 16, ks, lane);
    };
    auto fragB = [&](const char *t, int j, int ks) -> h8 {
        if constexpr (MI == 32) return frag<BN, TB, BK>(t, wn0 + j * 32, ks, lane);
        else return frag16<BN, TB, BK>(t, wn0 + j * 16, ks, lane);
    };

    static_assert(FETCH != 3 || (BK == 64 && 64 * NW == 2 * BM && BM == BN), "prefetch mapping: one line per thread");
    const char *junk = gsm + SMEM0 + wave * 256;
    // prefetch: the first half of the waves covers A's stage lines, the second half B's. The branch
    // is on a scalar (wave-uniform) value, so each wave issues exactly one prefetch load per stage,
    // which the vmcnt accounting of the loop relies on.
    const bool pf_a = __builtin_amdgcn_readfirstlane(wave) < NW / 2;
    auto prefetch = [&](int k0) {
        if (pf_a) prefetch_stage<BM, TA>(ab(k0), d.lda, m0, d.M, k0, tid, junk);
        else prefetch_stage<BN, TB>(bb(k0), d.ldb, n0, d.N, k0, tid - BM, junk);
    };
#pragma unroll
    for (int p = 0; p < NS - 1; p++) {
        const int kp = min(p, nkt - 1) * BK;
        if constexpr (FETCH >= 3) {
            fa.issue_asm(ab(kp), d.lda, kp, gsm_lds + p * STAGE, wave_u);
            fb.issue_asm(bb(kp), d.ldb, kp, gsm_lds + p * STAGE + ABYTES, wave_u);
        } else {
            fa.issue(ab(kp), d.lda, kp, gsm + p * STAGE, wave);
            fb.issue(bb(kp), d.ldb, kp, gsm + p * STAGE + ABYTES, wave);
        }
    }
    if constexpr (FETCH == 3) prefetch(min(NS - 1, nkt - 1) * BK);
    // Waits until stage kt has landed: its own loads are done once at most the younger stages' loads
    // (and, with prefetching, the one younger prefetch line) are still in flight; the barrier then
    // covers every wave's loads, and every wave has finished reading the buffer refilled next.
    auto stage_wait = [&]() {
        if constexpr (FETCH == 3) asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NS - 2) * PERSTAGE + 1) : "memory");
        else asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NS - 2) * PERSTAGE) : "memory");
        if constexpr (FETCH >= 3) lds_barrier();
        else __syncthreads();
    };
    // Fetch modes 2-4: right after the barrier that opens stage kt, refill the buffer consumed in
    // stage kt-1 with stage kt+NS-1 (clamped: the tail re-fetches the last stage into idle buffers,
    // keeping the number of loads in flight, and so the wait counts, the same in every iteration).
    auto issue_grouped = [&](int kt, bool all_modes = false) {
        char *nxt = gsm + ((kt + NS - 1) % NS) * STAGE;
        const int kn = min(kt + NS - 1, nkt - 1) * BK;
        if (FETCH >= 5 && !all_modes) {
            // mode 5 issues these between the MFMAs that follow
        } else if constexpr (FETCH == 2) {
            fa.issue(ab(kn), d.lda, kn, nxt, wave);
            fb.issue(bb(kn), d.ldb, kn, nxt + ABYTES, wave);
        } else if constexpr (FETCH >= 3) {
            const uint32_t nxt_lds = gsm_lds + ((kt + NS - 1) % NS) * STAGE;
            fa.issue_asm(ab(kn), d.lda, kn, nxt_lds, wave_u);
            fb.issue_asm(bb(kn), d.ldb, kn, nxt_lds + ABYTES, wave_u);
            if constexpr (FETCH == 3) prefetch(min(kt + NS, nkt - 1) * BK);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    h8 a[2][FA], b[2][FB];
    if constexpr (XB) {
        stage_wait();
        issue_grouped(0, true);
#pragma unroll
        for (int i = 0; i < FA; i++) a[0][i] = fragA(gsm, i, 0);
#pragma unroll
        for (int j = 0; j < FB; j++) b[0][j] = fragB(gsm + ABYTES, j, 0);
    }
    for (int kt = 0; kt < nkt; kt++) {
        const char *sa = gsm + (kt % NS) * STAGE, *sb = sa + ABYTES;
        char *nxt = gsm + ((kt + NS - 1) % NS) * STAGE;   // fetch modes 0 and 1 refill this buffer
        const int kn = min(kt + NS - 1, nkt - 1) * BK;
        if constexpr (!XB) {
            stage_wait();
            if constexpr (FETCH >= 2) issue_grouped(kt);
#pragma unroll
            for (int i = 0; i < FA; i++) a[0][i] = fragA(sa, i, 0);
#pragma unroll
            for (int j = 0; j < FB; j++) b[0][j] = fragB(sb, j, 0);
        }
        // Scheduling fences fix the issue order: the LDS reads of k-step s+1 go out as a group ahead
        // of the MFMAs of k-step s (their latency hides behind the MFMAs); the stage fetches are
        // spread evenly between the MFMAs (issued back to back they fill the vector-memory queue
        // and stall MFMA issue); MFMAs of different k-steps, which share accumulators, never mix.
        __builtin_amdgcn_sched_barrier(0);
        constexpr int NM = FA * FB;
        constexpr int PA = Fetch<BM, TA, BK, NW>::PER;
        constexpr int FPS = (PERSTAGE + KS - 1) / KS;                      // fetches per k-step
        constexpr bool SPREAD = FETCH == 1;
        if constexpr (FETCH == 0) {
            fa.issue(ab(kn), d.lda, kn, nxt, wave);
            fb.issue(bb(kn), d.ldb, kn, nxt + ABYTES, wave);
        }
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const int c = s & 1, n = c ^ 1;
            if (s + 1 < KS) {
                if constexpr (FETCH >= 6) __builtin_amdgcn_sched_barrier(0);   // one region per k-step
#pragma unroll
                for (int i = 0; i < FA; i++) a[n][i] = fragA(sa, i, s + 1);
#pragma unroll
                for (int j = 0; j < FB; j++) b[n][j] = fragB(sb, j, s + 1);
                if constexpr (FETCH < 6) __builtin_amdgcn_sched_barrier(0);
            } else if constexpr (XB) {
                // Open stage kt+1 now (KS is even, so its first fragments go to slot n = 0). In the
                // last iteration this reads a re-fetched copy of the last stage, which is unused. The
                // fence keeps the MFMAs of k-step s-1 ahead of the barrier.
                __builtin_amdgcn_sched_barrier(0);
                stage_wait();
                issue_grouped(kt + 1);
                const char *sa1 = gsm + ((kt + 1) % NS) * STAGE, *sb1 = sa1 + ABYTES;
#pragma unroll
                for (int i = 0; i < FA; i++) a[n][i] = fragA(sa1, i, 0);
#pragma unroll
                for (int j = 0; j < FB; j++) b[n][j] = fragB(sb1, j, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            // mode 5: the refill of stage kt's buffer with stage kt+NS, one DMA after every MPD MFMAs
            constexpr int MPD = NM >= PERSTAGE ? NM / PERSTAGE : 1;
            constexpr int DPM = NM >= PERSTAGE ? 1 : PERSTAGE / NM;
            static_assert(FETCH < 5 || MPD * PERSTAGE == NM || DPM * NM == PERSTAGE, "DMAs must spread evenly");
            const uint32_t refill_lds = gsm_lds + (kt % NS) * STAGE;
            const int kr = min(kt + NS, nkt - 1) * BK;
#pragma unroll
            for (int t = 0; t < NM; t++) {
                if constexpr (MI == 32)
                    acc[t / FN][t % FN] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c][t / FN], b[c][t % FN], acc[t / FN][t % FN], 0, 0, 0);
                else
                    acc4[t / FB][t % FB] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c][t / FB], b[c][t % FB], acc4[t / FB][t % FB], 0, 0, 0);
                if constexpr (FETCH >= 5) {
                    if (s == KS - 1 && t % MPD == MPD - 1) {
#pragma unroll
                        for (int q = 0; q < DPM; q++) {
                            const int f = (t / MPD) * DPM + q;
                            if (f < PA) fa.issue_one_asm(f, ab(kr), d.lda, kr, refill_lds, wave_u);
                            else fb.issue_one_asm(f - PA, bb(kr), d.ldb, kr, refill_lds + ABYTES, wave_u);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                if (SPREAD && t % (NM / FPS) == NM / FPS - 1) {
                    const int f = s * FPS + t / (NM / FPS);
                    if (f < PA) fa.issue_one(f, ab(kn), d.lda, kn, nxt, wave);
                    else if (f < PERSTAGE) fb.issue_one(f - PA, bb(kn), d.ldb, kn, nxt + ABYTES, wave);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if constexpr (FETCH == 7) {
                if (s + 1 < KS) {
                    // ds reads of k-step s+1 spread evenly: one after every NM/NR MFMAs (or RPM after
                    // each MFMA when there are more reads than MFMAs)
                    constexpr int NR = (TA ? 2 : 1) * FA + (TB ? 2 : 1) * FB;
                    constexpr int RPM = (NR + NM - 1) / NM;
                    constexpr int MPR = NR >= NM ? 1 : NM / NR;
                    constexpr int NG = (NR + RPM - 1) / RPM;
#pragma unroll
                    for (int q = 0; q < NG; q++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, MPR, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, RPM, 0);
                    }
                    if constexpr (NM > NG * MPR) __builtin_amdgcn_sched_group_barrier(0x008, NM - NG * MPR, 0);
                }
            }
            if constexpr (FETCH == 6) {
                if (s + 1 < KS) {
                    // ds reads of k-step s+1 (two per fragment for the transposing read): RPM after
                    // each of the first MFMAs, then the rest of the MFMAs
                    constexpr int NR = (TA ? 2 : 1) * FA + (TB ? 2 : 1) * FB;
                    constexpr int RPM = (NR + NM - 1) / NM;
                    constexpr int NMR = (NR + RPM - 1) / RPM;
#pragma unroll
                    for (int q = 0; q < NMR; q++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // one MFMA
                        __builtin_amdgcn_sched_group_barrier(0x100, RPM, 0);   // then RPM LDS reads
                    }
                    __builtin_amdgcn_sched_group_barrier(0x008, NM - NMR, 0);
                }
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // drain the tail re-fetches before LDS reuse

    const int mb = m0 + wm0, nb = n0 + wn0;
    // element r of lane l of 32x32 block (i, j) of the accumulators, for either MFMA shape
    auto accv = [&](int i, int j, int r) -> float {
        if constexpr (MI == 32) return acc[i][j][r];
        else return AccView16<FM, FN>{acc4}(i, j, r);
    };
    if constexpr (KG == 1) {
        if constexpr (MI == 32) {
            if (!fold.template run<FM, FN, 64 * NW>(acc, tid)) return;
        } else {
            static_assert(std::is_same<Fold, G16NoFold>::value, "MI 16 tiles have no split-K fold");
        }
    }
    if constexpr (KG > 1) {
        // The two k-groups split the finish: group g owns 32-row block g of each wave tile (which has
        // two). Each group hands the other group's block over through LDS (element e of lane l of
        // wave w at [w][e][l], conflict-free), adds the block it receives, and runs the epilogue on
        // its own block, so all waves of the workgroup take part in the epilogue traffic.
        static_assert(KG == 2 && FM == 2, "k-groups split the wave tile's two row blocks");
        constexpr int NE = FM * FN * 16;
        float *red = (float *)smem + wave * NE * 64 + lane;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {   // hand over the block the other group owns
                const float v = kg == 0 ? accv(1, j, r) : accv(0, j, r);
                red[(((1 - kg) * FN + j) * 16 + r) * 64] = v;
            }
        __syncthreads();
        // own block + the other group's partial of it (f32 addition is commutative, so the sum is the
        // same whichever group adds it)
        floatx16 mine[1][FN];
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float own = kg == 0 ? accv(0, j, r) : accv(1, j, r);
                mine[0][j][r] = own + red[((kg * FN + j) * 16 + r) * 64];
            }
        __syncthreads();   // the epilogue below reuses this LDS
        if constexpr (VEPI)
            epilogue_lds<EPI, half_t, 1, FN, MI>(d, mine, mb + kg * 32, nb, lane, smem + (kg * NW + wave) * (32 * 256));
        else
            epilogue_tile<EPI, half_t, 1, FN>(d, mine, mb + kg * 32, nb, lane);
        return;
    }
    if constexpr (VEPI) {
        // Epilogue through the (now idle) operand LDS: each wave owns FM*32 rows x 64 f32 columns.
        __syncthreads();
        if constexpr (MI == 32) epilogue_lds<EPI, half_t, FM, FN>(d, acc, mb, nb, lane, smem + wave * (WM * 256));
        else epilogue_lds_view<EPI, half_t, FM, FN, 16>(d, AccView16<FM, FN>{acc4}, mb, nb, lane, smem + wave * (WM * 256));
    } else {
        epilogue_tile<EPI, half_t, FM, FN>(d, acc, mb, nb, lane);
    }
}

template <int BM, int BN, int TA, int TB, int EPI, bool VEPI, int BK, int NS, int WVM, int WVN, int FETCH, bool XB, int KG,
          bool HL = false, int MI = 32>
__global__ __launch_bounds__(64 * WVM * WVN * KG) void gemm16_kernel(GemmDesc d) {
    __shared__ __attribute__((aligned(1024))) char smem[G16Smem<BM, BN, BK, NS, WVM, WVN, FETCH, KG>::SMEM];
    const int tiles_n = (d.N + BN - 1) / BN;
    const int tiles_m = (d.M + BM - 1) / BM;
    const int ntiles = tiles_m * tiles_n;
    int L = blockIdx.x;
    if ((ntiles & 7) == 0) L = (L & 7) * (ntiles >> 3) + (L >> 3);   // contiguous tile runs per XCD
    int m0, n0;
    g16_tile_origin(L, tiles_m, tiles_n, BM, BN, m0, n0);
    g16_tile<BM, BN, TA, TB, EPI, VEPI, BK, NS, WVM, WVN, FETCH, XB, KG, G16NoFold, HL, MI>(d, smem, m0, n0, 0, d.K, G16NoFold{});
}

template <int T>
static bool operand_ok(const void *p, long ld, int rows) {
    if (((uintptr_t)p & 15) || (ld % 8) || rows < 8) return false;
    // K-contiguous operands address each lane's row by a 32-bit byte offset from the stage base
    if (T == 0) return (long)rows * ld * 2 < (1l << 32);
    return (rows % 8) == 0;
}

// MI 16 variants have only the LDS-staged epilogue: a tile that needs the per-element one runs the
// variant's MI 32 form.
template <int BM, int WVM, int WVN, int BK, int NS, int FETCH, bool XB, int KG, int TA, int TB, int EPI, bool HL = false, int MI = 32>
static hipError_t launch(const GemmDesc &d, hipStream_t s) {
    int tiles = ((d.M + BM - 1) / BM) * ((d.N + BM - 1) / BM);
    const uintptr_t a = (uintptr_t)d.C | (uintptr_t)d.aux | (uintptr_t)d.bias | (uintptr_t)d.W32 |
                        (uintptr_t)d.W16 | (uintptr_t)d.gout | (uintptr_t)d.C2;
    const bool vepi = d.M % BM == 0 && d.N % BM == 0 && d.ldc % 4 == 0 && d.ldaux % 4 == 0 && (a & 15) == 0;
    constexpr int NT = 64 * WVM * WVN * KG;
    if (vepi) hipLaunchKernelGGL((gemm16_kernel<BM, BM, TA, TB, EPI, true, BK, NS, WVM, WVN, FETCH, XB, KG, HL, MI>), dim3(tiles), dim3(NT), 0, s, d);
    else hipLaunchKernelGGL((gemm16_kernel<BM, BM, TA, TB, EPI, false, BK, NS, WVM, WVN, FETCH, XB, KG, HL>), dim3(tiles), dim3(NT), 0, s, d);
    return hipGetLastError();
}

// Variants (GemmDesc::variant): tile BM (square), wave layout WVM x WVN, k per stage BK, stages in
// flight NS, fetch mode, cross-barrier prefetch XB, k-groups KG.
template <int V> struct Var;
#define AH_G16_VARM(V, BM_, WVM_, WVN_, BK_, NS_, FETCH_, XB_, KG_, MI_)                               \
    template <> struct Var<V> {                                                                      \
        static constexpr int BM = BM_, WVM = WVM_, WVN = WVN_, BK = BK_, NS = NS_, FETCH = FETCH_, KG = KG_; \
        static constexpr int MI = MI_;                                                               \
        static constexpr bool XB = XB_;                                                              \
    };
#define AH_G16_VAR(V, BM_, WVM_, WVN_, BK_, NS_, FETCH_, XB_, KG_) AH_G16_VARM(V, BM_, WVM_, WVN_, BK_, NS_, FETCH_, XB_, KG_, 32)
AH_G16_VAR(1, 128, 2, 2, 64, 2, 0, false, 1)
AH_G16_VAR(2, 256, 2, 2, 64, 2, 1, false, 1)   // one wave per SIMD
AH_G16_VAR(3, 256, 4, 2, 64, 2, 1, false, 1)   // two waves per SIMD, 64x128 per wave
AH_G16_VAR(4, 256, 4, 2, 64, 2, 2, false, 1)
AH_G16_VAR(5, 128, 2, 2, 64, 2, 2, false, 1)
AH_G16_VAR(6, 256, 2, 2, 64, 2, 2, false, 1)
AH_G16_VAR(7, 256, 4, 2, 32, 5, 2, false, 1)   // 160 KiB of stages
AH_G16_VAR(8, 256, 4, 2, 64, 2, 3, false, 1)
AH_G16_VAR(9, 128, 2, 2, 64, 2, 3, false, 1)
AH_G16_VAR(10, 128, 2, 2, 64, 2, 3, false, 2)
AH_G16_VAR(11, 128, 2, 2, 64, 2, 2, false, 2)
AH_G16_VAR(12, 256, 4, 2, 32, 4, 4, true, 1)
AH_G16_VAR(13, 256, 4, 2, 64, 2, 4, true, 1)
AH_G16_VAR(14, 128, 2, 2, 64, 4, 4, true, 1)
AH_G16_VAR(15, 128, 2, 2, 64, 2, 4, true, 2)
AH_G16_VAR(16, 256, 4, 2, 32, 5, 4, true, 1)
AH_G16_VAR(17, 256, 4, 2, 64, 2, 3, true, 1)
AH_G16_VAR(18, 256, 4, 2, 32, 4, 4, false, 1)
AH_G16_VAR(19, 128, 2, 2, 64, 3, 4, true, 1)
AH_G16_VAR(20, 256, 2, 2, 64, 2, 4, true, 1)   // one wave per SIMD, 128x128 per wave
AH_G16_VAR(21, 256, 2, 2, 32, 4, 4, true, 1)
AH_G16_VAR(22, 256, 2, 2, 64, 2, 5, true, 1)
AH_G16_VAR(23, 256, 4, 2, 64, 2, 5, true, 1)
AH_G16_VAR(24, 128, 2, 2, 64, 3, 5, true, 1)
AH_G16_VAR(25, 128, 2, 2, 64, 2, 5, true, 2)
AH_G16_VAR(26, 256, 2, 2, 64, 2, 6, true, 1)
AH_G16_VAR(27, 256, 4, 2, 64, 2, 6, true, 1)
AH_G16_VAR(28, 128, 2, 2, 64, 2, 6, true, 2)
AH_G16_VAR(29, 256, 2, 2, 64, 2, 7, true, 1)
AH_G16_VAR(30, 256, 4, 2, 64, 2, 7, true, 1)
AH_G16_VAR(31, 128, 2, 2, 64, 2, 7, true, 2)
// 16x16x32 MFMAs (MI 16): under sustained load on varied data the 16x16x32 instruction sustains more
// of its nominal rate than 32x32x16 before the power limit lowers the clock
AH_G16_VARM(32, 256, 4, 2, 64, 2, 6, true, 1, 16)
AH_G16_VARM(33, 256, 4, 2, 64, 2, 7, true, 1, 16)
AH_G16_VARM(34, 256, 4, 2, 64, 2, 4, true, 1, 16)
AH_G16_VARM(35, 128, 2, 2, 64, 2, 5, true, 2, 16)
AH_G16_VARM(36, 128, 2, 2, 64, 2, 4, true, 2, 16)
AH_G16_VARM(37, 128, 2, 2, 64, 2, 7, true, 2, 16)
AH_G16_VARM(38, 128, 2, 2, 64, 2, 6, true, 2, 16)
AH_G16_VARM(39, 256, 4, 2, 64, 2, 5, true, 1, 16)
#undef AH_G16_VAR
#undef AH_G16_VARM
constexpr int kMaxVariant = 39;

template <int V, int TA, int TB>
static hipError_t run_epi(const GemmDesc &d, hipStream_t s) {
    using P = Var<V>;
    if (d.A2) {
        // two-plane contractions are instantiated for the adjoint products of the f32-adjoint MLP step:
        // dX with the ReLU mask (A K-contiguous, B MN-contiguous) and dW with the SGD update (both
        // MN-contiguous)
        if constexpr (TA == 0 && TB == 1) {
            if (d.epi == EPI_MASK) return launch<P::BM, P::WVM, P::WVN, P::BK, P::NS, P::FETCH, P::XB, P::KG, 0, 1, EPI_MASK, true, P::MI>(d, s);
        }
        if constexpr (TA == 1 && TB == 1) {
            if (d.epi == EPI_SGD) return launch<P::BM, P::WVM, P::WVN, P::BK, P::NS, P::FETCH, P::XB, P::KG, 1, 1, EPI_SGD, true, P::MI>(d, s);
        }
        return hipErrorInvalidValue;
    }
#define AH_G16_L(E) launch<P::BM, P::WVM, P::WVN, P::BK, P::NS, P::FETCH, P::XB, P::KG, TA, TB, E, false, P::MI>(d, s)
    switch (d.epi) {
        case EPI_STORE: return AH_G16_L(EPI_STORE);
        case EPI_BIAS: return AH_G16_L(EPI_BIAS);
        case EPI_BIAS_RELU: return AH_G16_L(EPI_BIAS_RELU);
        case EPI_MSE: return AH_G16_L(EPI_MSE);
        case EPI_MASK: return AH_G16_L(EPI_MASK);
        case EPI_SGD: return AH_G16_L(EPI_SGD);
        default: return hipErrorInvalidValue;
    }
#undef AH_G16_L
}

// Launches variant V for every operand layout and epilogue.
template <int V>
hipError_t run_variant(const GemmDesc &d, hipStream_t s) {
    switch (d.ta * 2 + d.tb) {
        case 0: return run_epi<V, 0, 0>(d, s);
        case 1: return run_epi<V, 0, 1>(d, s);
        case 2: return run_epi<V, 1, 0>(d, s);
        default: return run_epi<V, 1, 1>(d, s);
    }
}

}  // namespace g16
}  // namespace ah
