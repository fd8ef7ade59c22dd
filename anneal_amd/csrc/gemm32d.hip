// gemm32d.hip — f32 MFMA contraction for gfx950 with direct global->LDS stages.
//
// Block tile BM x BM, 4 wave64s in a 2x2 arrangement, each wave owning a (BM/2)^2 sub-tile of 32x32
// v_mfma_f32_32x32x2f32 blocks. K advances in LDS stages of BK floats, NS stages in flight: every
// operand tile is fetched with global_load_lds_dwordx4 (each lane's 16 bytes land at the LDS base +
// 16 * lane), so loads of later stages are in flight while a stage is contracted and no VGPRs or
// ds_write instructions are spent on staging (the register-staged kernel in gemm.hip waits on each
// stage's loads before storing them to LDS). The fetch order is chosen so that the LDS image is
// conflict-free for the fragment reads:
//   K-contiguous operand ([rows][K]): rows of BK floats; BK = 32: pairs of 128-byte rows form 256-byte
//     super-rows whose 16-byte slots are XOR-swizzled by the super-row index; BK = 64: 256-byte rows
//     whose slots are XOR-swizzled by the row index. Fragments are ds_read_b128 (4 consecutive k).
//   MN-contiguous operand ([K][rows]): k-rows in the stored orientation, the 16-byte slots of k-rows
//     with bit 2 of k set XORed by 8, so that the two k-rows one fragment read touches (k and k+4) sit
//     32 banks apart. Fragments are ds_read_b32 (one k per lane).
// Each 8-k step accumulates, for q = 0..3, the products of k = 8s+q (lanes 0-31) and k = 8s+4+q
// (lanes 32-63) in one MFMA, over k in increasing order: the order of the register-staged kernel with
// one k-group and no split of K, so the two give the same bits for every layout (tested). Wave tiles of
// a single 32x32 block keep two accumulator banks (elements 0 and 2 of a chunk in one, 1 and 3 in the
// other, added at the end) as the register-staged kernel does.
#include "ah_common.h"
#include "gemm.h"
#include "gemm_epi.h"

namespace ah {

// Workgroups splitting K per tile: GemmDesc::splits when above 1, the K range a whole number of stages
// per split and the device's split-K workspace large enough; else 1.
int gemm32d_splits(const GemmDesc &d, int bm, int bk) {
    int sp = d.splits > 16 ? 16 : d.splits;
    if (sp <= 1 || !d.sk_sync || !d.sk_part) return 1;
    const long tiles = (long)((d.M + bm - 1) / bm) * ((d.N + bm - 1) / bm);
    if (tiles > kSplitKMaxTiles || d.K % (bk * sp) || tiles * sp * bm * bm > d.sk_cap) return 1;
    return sp;
}

namespace g32 {

// Byte offset of 16-byte chunk c (k = 4c .. 4c+3) of row r in a K-contiguous stage of BK floats per row.
template <int BK>
__device__ __forceinline__ int koff(int r, int c) {
    if constexpr (BK == 32) {
        const int q = r >> 1;
        return q * 256 + (((((r & 1) << 3) | c) ^ (q & 15)) << 4);
    } else {
        static_assert(BK == 64, "K-contiguous stages hold 32 or 64 floats per row");
        return r * 256 + ((c ^ (r & 15)) << 4);
    }
}
// Byte offset of chunk c (rows 4c .. 4c+3) of k-row k in an MN-contiguous stage of R floats per k-row.
template <int R>
__device__ __forceinline__ int mnoff(int k, int c) {
    return k * (R * 4) + ((c ^ (((k >> 2) & 1) << 3)) << 4);
}

// The stage slot S (16 bytes, LDS byte 16 * S of the operand's stage image) -> the global element it
// holds, as (row or k-row, chunk) of the stored layout; the inverses of koff / mnoff.
template <int R, int T, int BK>
__device__ __forceinline__ void slot_src(int S, int &row, int &chunk) {
    if constexpr (T == 0) {
        if constexpr (BK == 32) {
            const int q = S >> 4, x = (S & 15) ^ (q & 15);
            row = 2 * q + (x >> 3);
            chunk = x & 7;
        } else {
            row = S >> 4;
            chunk = (S & 15) ^ (row & 15);
        }
    } else {
        constexpr int CHR = R / 4;   // chunks per k-row
        row = S / CHR;               // k-row
        chunk = (S % CHR) ^ (((row >> 2) & 1) << 3);
    }
}

// One 16-byte-per-lane global->LDS DMA: wave-uniform base in SGPRs plus the lane's 32-bit offset, the
// LDS destination in M0. Issued from inline asm, so the compiler's wait-count model does not see it and
// adds no conservative waits; the kernel orders these loads with its own s_waitcnt vmcnt. The compiler
// emits nothing that reads M0 in this kernel.
__device__ __forceinline__ void dma16(uint32_t voff, const char *sbase, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
                 : "memory", "m0");
}
// Workgroup barrier that waits only for this wave's LDS reads (a __syncthreads would also wait for the
// stages still meant to be in flight).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Per-lane byte offsets, relative to the tile's origin in the stored array, of the 1 KiB blocks of one
// operand stage this wave fetches (stage-independent; a stage adds k0 to the base).
template <int R, int T, int BK>
struct Fetch {
    static constexpr int NB = R * BK * 4 / 1024;   // 1 KiB blocks per stage
    static constexpr int PER = NB / 4;             // per wave
    static_assert(PER * 4 == NB, "stage blocks split evenly over the 4 waves");
    uint32_t off[PER];
    // r0: the tile's first row (K-contiguous) or column (MN-contiguous); rmax: the operand's rows (M or N)
    __device__ __forceinline__ void init(long ld, int r0, int rmax, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int S = (wave * PER + j) * 64 + lane;
            int row, chunk;
            slot_src<R, T, BK>(S, row, chunk);
            if constexpr (T == 0) {
                const int r = min(r0 + row, rmax - 1) - r0;          // ragged rows re-read the last row
                off[j] = (uint32_t)(((long)r * ld + chunk * 4) * 4);
            } else {
                const int m = min(r0 + chunk * 4, rmax - 4) - r0;    // ragged columns re-read the last chunk
                off[j] = (uint32_t)(((long)row * ld + m) * 4);
            }
        }
    }
    // this wave's loads of the stage at k0 into the operand image at LDS address img
    __device__ __forceinline__ void issue(const char *tile_base, long ld, int k0, uint32_t img, int wave) const {
        const char *base = tile_base + (T == 0 ? (long)k0 * 4 : (long)k0 * ld * 4);
#pragma unroll
        for (int j = 0; j < PER; j++) dma16(off[j], base, img + (uint32_t)((wave * PER + j) * 1024));
    }
};

typedef float f4 __attribute__((ext_vector_type(4)));

// The fragment of 32 rows (or columns) at r of 8-k step s: element q of lane l is k = 8s + 4(l/32) + q.
template <int R, int T, int BK>
__device__ __forceinline__ f4 frag(const char *img, int r, int s, int lane) {
    if constexpr (T == 0) {
        return *(const f4 *)(img + koff<BK>(r + (lane & 31), 2 * s + (lane >> 5)));
    } else {
        const int m = r + (lane & 31), k = 8 * s + 4 * (lane >> 5);
        f4 v;
#pragma unroll
        for (int q = 0; q < 4; q++) v[q] = *(const float *)(img + mnoff<R>(k + q, m >> 2) + (m & 3) * 4);
        return v;
    }
}

template <int BM, int BK, int NS>
struct Smem {
    static constexpr int IMG = BM * BK * 4;         // one operand's stage image
    static constexpr int STAGE = 2 * IMG;
    static constexpr int SMEM = NS * STAGE;
};

template <int BM, int TA, int TB, int EPI, int BK, int NS>
__global__ __launch_bounds__(256) void gemm32d_kernel(GemmDesc d) {
    using SM = Smem<BM, BK, NS>;
    constexpr int WM = BM / 2, FM = WM / 32;
    constexpr int ST = BK / 8;                      // 8-k steps per stage
    constexpr bool ILP2 = FM == 1;
    constexpr int PERSTAGE = Fetch<BM, TA, BK>::PER + Fetch<BM, TB, BK>::PER;
    __shared__ __attribute__((aligned(1024))) char smem[SM::SMEM];

    const int tiles_n = (d.N + BM - 1) / BM, tiles_m = (d.M + BM - 1) / BM, ntiles = tiles_m * tiles_n;
    int L = blockIdx.x;
    // the register-staged kernel's tile order: XCD-aware runs of tiles, then groups of 4 tile-rows
    if ((ntiles & 7) == 0) L = (L & 7) * (ntiles >> 3) + (L >> 3);
    constexpr int G = 4;
    const int group = L / (G * tiles_n), gm0 = group * G, gsz = min(G, tiles_m - gm0);
    const int rem = L - group * G * tiles_n;
    const int m0 = (gm0 + rem % gsz) * BM, n0 = (rem / gsz) * BM;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WM;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)smem;

    Fetch<BM, TA, BK> fa;
    Fetch<BM, TB, BK> fb;
    fa.init(d.lda, m0, d.M, wave, lane);
    fb.init(d.ldb, n0, d.N, wave, lane);
    // split-K: the gridDim.y workgroups of a tile each contract one K / gridDim.y range (whole stages)
    const int nsplit = gridDim.y, split = blockIdx.y;
    const int nk = d.K / BK / nsplit;
    const long kb = (long)split * nk * BK;
    const char *Ab = (const char *)d.A + (TA == 0 ? (long)m0 * d.lda * 4 + kb * 4 : (long)m0 * 4 + kb * d.lda * 4);
    const char *Bb = (const char *)d.B + (TB == 0 ? (long)n0 * d.ldb * 4 + kb * 4 : (long)n0 * 4 + kb * d.ldb * 4);

    floatx16 acc[FM][FM], acc2[FM][FM];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FM; j++) acc[i][j] = acc2[i][j] = (floatx16){};

    // stages 0 .. NS-2 in flight; later issues past the last stage re-fetch it (into buffers no longer
    // read), so every iteration issues the same number of loads and the wait counts stay fixed
#pragma unroll
    for (int p = 0; p < NS - 1; p++) {
        const int kp = min(p, nk - 1) * BK;
        fa.issue(Ab, d.lda, kp, lds0 + p * SM::STAGE, wave);
        fb.issue(Bb, d.ldb, kp, lds0 + p * SM::STAGE + SM::IMG, wave);
    }
    for (int kt = 0; kt < nk; kt++) {
        // stage kt has landed once at most the NS-2 younger stages' loads are outstanding; after the
        // barrier every wave's part of it has, and every wave is done with the buffer refilled next
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NS - 2) * PERSTAGE) : "memory");
        lds_barrier();
        {
            const int buf = (kt + NS - 1) % NS, kn = min(kt + NS - 1, nk - 1) * BK;
            fa.issue(Ab, d.lda, kn, lds0 + buf * SM::STAGE, wave);
            fb.issue(Bb, d.ldb, kn, lds0 + buf * SM::STAGE + SM::IMG, wave);
        }
        const char *sa = smem + (kt % NS) * SM::STAGE, *sb = sa + SM::IMG;
        f4 a[2][FM], b[2][FM];
#pragma unroll
        for (int i = 0; i < FM; i++) a[0][i] = frag<BM, TA, BK>(sa, wm0 + 32 * i, 0, lane);
#pragma unroll
        for (int j = 0; j < FM; j++) b[0][j] = frag<BM, TB, BK>(sb, wn0 + 32 * j, 0, lane);
#pragma unroll
        for (int s = 0; s < ST; s++) {
            const int cb = s & 1, nb = cb ^ 1;
            if (s + 1 < ST) {
#pragma unroll
                for (int i = 0; i < FM; i++) a[nb][i] = frag<BM, TA, BK>(sa, wm0 + 32 * i, s + 1, lane);
#pragma unroll
                for (int j = 0; j < FM; j++) b[nb][j] = frag<BM, TB, BK>(sb, wn0 + 32 * j, s + 1, lane);
            }
            __builtin_amdgcn_sched_barrier(0);   // the next step's reads ahead of this step's MFMAs
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FM; j++) {
                    const f4 &x = a[cb][i], &y = b[cb][j];
                    if constexpr (ILP2) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(x[0], y[0], acc[i][j], 0, 0, 0);
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(x[1], y[1], acc2[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(x[2], y[2], acc[i][j], 0, 0, 0);
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(x[3], y[3], acc2[i][j], 0, 0, 0);
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; q++)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(x[q], y[q], acc[i][j], 0, 0, 0);
                    }
                }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // the tail re-fetches must land before the workgroup's LDS can be reused
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if constexpr (ILP2) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FM; j++) acc[i][j] += acc2[i][j];
    }
    if (nsplit > 1) {
        // The register-staged kernel's split-K finish: every split stores its partial with 16-byte sc1
        // buffer stores (written through, coherent across the XCDs' L2s), waits for them, and takes a
        // ticket from the tile's arrival counter (acquire-release); the split drawing the last ticket adds
        // all partials in split order (its own from registers), resets the counter and runs the epilogue.
        // Partial layout: 16-byte chunk c of thread t at byte 16 * (c * 256 + t) of its split.
        constexpr int NC = FM * FM * 4, PART = NC * 256 * 16, SC1 = 16;
        typedef unsigned u4 __attribute__((ext_vector_type(4)));
        const int tile = (m0 / BM) * tiles_n + n0 / BM;
        int *const count = d.sk_sync + 2 * tile;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            d.sk_part + (long)tile * nsplit * (PART / 4), (short)0, nsplit * PART, 0x00020000);
        __shared__ int ticket;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const floatx16 &a = acc[c / (FM * 4)][(c / 4) % FM];
            const int e = (c % 4) * 4;
            const floatx4 v = {a[e], a[e + 1], a[e + 2], a[e + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, split * PART + (c * 256 + tid) * 16, 0, SC1);
            // wait states before the store's data registers may be rewritten (a compiler-placed VALU write
            // two instructions behind a 16-byte store has reached memory in kernels of this library)
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_nop 4" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) ticket = ticket_take(count);
        __syncthreads();
        if (ticket != nsplit - 1) return;
#pragma unroll
        for (int bl = 0; bl < FM * FM; bl++) {
            floatx16 &a = acc[bl / FM][bl % FM];
            floatx4 sum[4];
            for (int q = 0; q < nsplit; q++) {
                floatx4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    if (q == split) v[u] = (floatx4){a[4 * u], a[4 * u + 1], a[4 * u + 2], a[4 * u + 3]};
                    else v[u] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, q * PART + ((bl * 4 + u) * 256 + tid) * 16, 0, SC1));
                }
#pragma unroll
                for (int u = 0; u < 4; u++) sum[u] = q == 0 ? v[u] : sum[u] + v[u];
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int x = 0; x < 4; x++) a[4 * u + x] = sum[u][x];
        }
        if (tid == 0) __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // next launch
    }
    epilogue_tile<EPI, float, FM, FM>(d, acc, m0 + wm0, n0 + wn0, lane);
}

template <int BM, int BK, int NS, int TA, int TB, int EPI>
static hipError_t launch(const GemmDesc &d, hipStream_t s) {
    const int tiles = ((d.M + BM - 1) / BM) * ((d.N + BM - 1) / BM);
    hipLaunchKernelGGL((gemm32d_kernel<BM, TA, TB, EPI, BK, NS>), dim3(tiles, gemm32d_splits(d, BM, BK)), dim3(256), 0, s, d);
    return hipGetLastError();
}

template <int BM, int BK, int NS, int TA, int TB>
static hipError_t launch_epi(const GemmDesc &d, hipStream_t s) {
    switch (d.epi) {
        case EPI_STORE: return launch<BM, BK, NS, TA, TB, EPI_STORE>(d, s);
        case EPI_BIAS: return launch<BM, BK, NS, TA, TB, EPI_BIAS>(d, s);
        case EPI_BIAS_RELU: return launch<BM, BK, NS, TA, TB, EPI_BIAS_RELU>(d, s);
        case EPI_MASK:
            if constexpr (BM == 64) return launch<BM, BK, NS, TA, TB, EPI_MASK>(d, s);
            else return hipErrorInvalidValue;
        case EPI_SGD:
            if constexpr (BM == 64) return launch<BM, BK, NS, TA, TB, EPI_SGD>(d, s);
            else return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

template <int BM, int BK, int NS>
static hipError_t launch_layout(const GemmDesc &d, hipStream_t s) {
    switch (d.ta * 2 + d.tb) {
        case 0: return launch_epi<BM, BK, NS, 0, 0>(d, s);
        case 1: return launch_epi<BM, BK, NS, 0, 1>(d, s);
        case 2: return launch_epi<BM, BK, NS, 1, 0>(d, s);
        default: return launch_epi<BM, BK, NS, 1, 1>(d, s);
    }
}

}  // namespace g32

bool gemm32d_config(int tile, int *bm, int *bk, int *ns) {
    switch (tile) {
        case kGemm32dBase + 0: *bm = 64; *bk = 64; *ns = 3; return true;
        case kGemm32dBase + 1: *bm = 64; *bk = 64; *ns = 4; return true;
        case kGemm32dBase + 2: *bm = 64; *bk = 32; *ns = 4; return true;
        case kGemm32dBase + 3: *bm = 128; *bk = 32; *ns = 4; return true;
        case kGemm32dBase + 4: *bm = 128; *bk = 64; *ns = 2; return true;
        default: return false;
    }
}

bool gemm32d_ok(const GemmDesc &d, int bm, int bk) {
    auto operand_ok = [&](const void *p, long ld, int t, int rows) {
        if (((uintptr_t)p & 15) || ld % 4) return false;
        if (t == 1 && rows % 4) return false;                        // 16-byte chunks of a k-row
        // per-lane offsets are 32-bit: a stage spans bm rows (K-contiguous) or bk k-rows (MN-contiguous)
        return (double)(t == 0 ? bm : bk) * (double)ld * 4.0 < 4294967296.0;
    };
    // 128-wide tiles take the store and bias epilogues only: with the ReLU-mask or SGD epilogue (16 loads
    // per lane in flight per 32x32 block) they run out of scalar registers and spill them to VGPR lanes
    if (bm == 128 && (d.epi == EPI_MASK || d.epi == EPI_SGD)) return false;
    return d.dtype == GEMM_F32 && d.epi != EPI_MSE && !d.A2 && !d.C2 && d.K > 0 && d.K % bk == 0 &&
           d.M >= 4 && d.N >= 4 && operand_ok(d.A, d.lda, d.ta, d.M) && operand_ok(d.B, d.ldb, d.tb, d.N);
}

hipError_t gemm32d_launch(const GemmDesc &d, hipStream_t s) {
    int bm, bk, ns;
    if (!gemm32d_config(d.tile, &bm, &bk, &ns) || !gemm32d_ok(d, bm, bk)) return hipErrorInvalidValue;
    switch (d.tile - kGemm32dBase) {
        case 0: return g32::launch_layout<64, 64, 3>(d, s);
        case 1: return g32::launch_layout<64, 64, 4>(d, s);
        case 2: return g32::launch_layout<64, 32, 4>(d, s);
        case 3: return g32::launch_layout<128, 32, 4>(d, s);
        default: return g32::launch_layout<128, 64, 2>(d, s);
    }
}

}  // namespace ah
