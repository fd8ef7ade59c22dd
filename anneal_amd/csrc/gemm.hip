// gemm.hip — LDS-staged MFMA contraction templates for gfx950 (CDNA4).
//
// Block tile BM x BN, 256 threads = 4 wave64s in a 2x2 arrangement, each wave owning a
// (BM/2) x (BN/2) sub-tile built from 32x32 MFMA blocks (f16: v_mfma_f32_32x32x16_f16,
// f32: v_mfma_f32_32x32x2f32). K advances in stages of 8 16-byte chunks per row (64 halves or
// 32 floats); two LDS stages are double-buffered so global loads of stage k+1 overlap the MFMAs of
// stage k. LDS rows are 128 B, paired into XOR-swizzled 256-byte super-rows (see lds_off).
// This generic path serves f32 operands and f16 shapes the direct-to-LDS kernel (gemm16.hip) rejects.
//
// Operands stored MN-contiguous ([K][M] / [K][N]) are transposed on the way into LDS: each
// thread loads a VEC x VEC sub-block with VEC coalesced 16-byte loads and writes VEC K-contiguous
// 16-byte rows, so the MFMA fragment reads are identical for every layout.
//
// Accumulation is f32 for both input types, matching the reference's f32 accumulator for f16
// reduces (codegen/lower.go:667-716); products of f16 inputs are exact in f32.
#include "ah_common.h"
#include "gemm.h"
#include "gemm_epi.h"

namespace ah {

constexpr int kThreads = 256;

// Two 128-byte rows form a 256-byte super-row whose 16-byte slots are XOR-swizzled by the super-row
// index: ds_read_b128 fragment reads (16 consecutive rows, one chunk) and the row-major stores hit 16
// distinct slots of the 64-bank LDS.
__device__ __forceinline__ int lds_off(int r, int c) {
    const int q = r >> 1;
    return q * 256 + (((((r & 1) << 3) | c) ^ (q & 15)) << 4);
}

template <typename T>
struct Mfma;

template <>
struct Mfma<half_t> {
    static constexpr int VEC = 8;
    typedef half_t vec_t __attribute__((ext_vector_type(8)));
    __device__ static __forceinline__ void mma(const vec_t &a, const vec_t &b, floatx16 &c) {
        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mfma<float> {
    static constexpr int VEC = 4;
    typedef float vec_t __attribute__((ext_vector_type(4)));
    // Lanes 0-31 hold k = 4c+q of chunk c, lanes 32-63 those of chunk c+1; the q-th MFMA
    // contracts element q of both halves. A and B use the same assignment, so the sum covers
    // each k exactly once.
    __device__ static __forceinline__ void mma(const vec_t &a, const vec_t &b, floatx16 &c) {
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0], b[0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[1], b[1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[2], b[2], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[3], b[3], c, 0, 0, 0);
    }
    // Two independent chains (elements 0,2 into c and 1,3 into c2): a wave holding a single 32x32
    // accumulator would otherwise issue four dependent 16-pass MFMAs back to back.
    __device__ static __forceinline__ void mma2(const vec_t &a, const vec_t &b, floatx16 &c, floatx16 &c2) {
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0], b[0], c, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[1], b[1], c2, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[2], b[2], c, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[3], b[3], c2, 0, 0, 0);
    }
};

// Guarded element-wise fill of one 16-byte chunk (slow path for unaligned / ragged shapes).
template <typename T>
__device__ __forceinline__ u32x4 load_chunk_guarded(const T *p, long step, int n_valid) {
    constexpr int VEC = 16 / sizeof(T);
    T tmp[VEC];
#pragma unroll
    for (int e = 0; e < VEC; e++) tmp[e] = (e < n_valid) ? p[e * step] : (T)0;
    u32x4 r;
    __builtin_memcpy(&r, tmp, 16);
    return r;
}

// Operand tile R rows x (8 chunks) from a K-contiguous array [rows][K].
template <typename T, int R>
struct LoadK {
    static constexpr int VEC = 16 / sizeof(T);
    static constexpr int PER = R * 8 / kThreads;
    u32x4 v[PER];
    __device__ __forceinline__ void load(const T *p, long ld, int r0, int rmax, int k0, int K, bool vec_ok, int tid) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            int id = tid + kThreads * i;
            int r = id >> 3, c = id & 7;
            int gr = r0 + r, gk = k0 + c * VEC;
            if (gr < rmax && gk < K) {
                const T *src = p + (long)gr * ld + gk;
                if (vec_ok) v[i] = *(const u32x4 *)src;
                else v[i] = load_chunk_guarded<T>(src, 1, K - gk);
            } else {
                v[i] = (u32x4){0, 0, 0, 0};
            }
        }
    }
    __device__ __forceinline__ void store(char *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            int id = tid + kThreads * i;
            *(u32x4 *)(lds + lds_off(id >> 3, id & 7)) = v[i];
        }
    }
};

// Operand tile from an MN-contiguous array [K][rows]: VEC x VEC sub-blocks, transposed in registers.
template <typename T, int R>
struct LoadMN {
    static constexpr int VEC = 16 / sizeof(T);
    static constexpr int RB = R / VEC;                 // sub-blocks along the row axis
    static constexpr int NSUB = 8 * RB;
    static constexpr int PER = (NSUB + kThreads - 1) / kThreads;
    u32x4 v[PER][VEC];
    __device__ __forceinline__ void load(const T *p, long ld, int r0, int rmax, int k0, int K, bool vec_ok, int tid) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            int id = tid + kThreads * i;
            int kb = id / RB, rb = id % RB;
            int gr = r0 + rb * VEC;
#pragma unroll
            for (int kk = 0; kk < VEC; kk++) {
                int gk = k0 + kb * VEC + kk;
                if (id < NSUB && gk < K && gr < rmax) {
                    const T *src = p + (long)gk * ld + gr;
                    if (vec_ok && gr + VEC <= rmax) v[i][kk] = *(const u32x4 *)src;
                    else v[i][kk] = load_chunk_guarded<T>(src, 1, rmax - gr);
                } else {
                    v[i][kk] = (u32x4){0, 0, 0, 0};
                }
            }
        }
    }
    __device__ __forceinline__ void store(char *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            int id = tid + kThreads * i;
            if (id >= NSUB) continue;
            int kb = id / RB, rb = id % RB;
            T in[VEC][VEC];
#pragma unroll
            for (int kk = 0; kk < VEC; kk++) __builtin_memcpy(in[kk], &v[i][kk], 16);
#pragma unroll
            for (int j = 0; j < VEC; j++) {
                T out[VEC];
#pragma unroll
                for (int kk = 0; kk < VEC; kk++) out[kk] = in[kk][j];
                u32x4 w;
                __builtin_memcpy(&w, out, 16);
                *(u32x4 *)(lds + lds_off(rb * VEC + j, kb)) = w;
            }
        }
    }
};

template <typename T, int R, int TR>
struct Loader;
template <typename T, int R>
struct Loader<T, R, 0> : LoadK<T, R> {};
template <typename T, int R>
struct Loader<T, R, 1> : LoadMN<T, R> {};

// KG: k-groups. The workgroup holds KG sets of 4 waves on the same tile; group g contracts the K
// chunks [g*nkg, (g+1)*nkg) (chunks past K load as zeros, so every group runs the same number of
// iterations and barriers), and groups 1..KG-1 hand their accumulators to group 0 through LDS, which
// adds them in group order (deterministic) and runs the epilogue. Small-output, long-K contractions
// (config 1's 64x128x784, config 4's small batches) get KG times the waves per tile.
template <typename T, int BM, int BN, int TA, int TB, int EPI, int KG>
__global__ __launch_bounds__(kThreads * KG) void gemm_kernel(GemmDesc d) {
    using MF = Mfma<T>;
    using vec_t = typename MF::vec_t;
    constexpr int VEC = MF::VEC;
    constexpr int BK = 8 * VEC;
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
    constexpr int STAGE = (BM + BN) * 128;
    constexpr int SMEM_K = KG * 2 * STAGE;
    constexpr int SMEM_R = (KG - 1) * BM * BN * 4;
    __shared__ __attribute__((aligned(16))) char smem[SMEM_K > SMEM_R ? SMEM_K : SMEM_R];

    const int tiles_n = (d.N + BN - 1) / BN;
    const int tiles_m = (d.M + BM - 1) / BM;
    const int ntiles = tiles_m * tiles_n;
    int L = blockIdx.x;
    // XCD-aware remap: workgroups are dealt round-robin over the 8 XCDs; give each XCD a
    // contiguous run of logical tiles so its L2 holds a compact block of A rows and B rows.
    if ((ntiles & 7) == 0) L = (L & 7) * (ntiles >> 3) + (L >> 3);
    // Grouped order: 4 tile-rows sweep all tile-columns before moving on.
    constexpr int G = 4;
    int group = L / (G * tiles_n);
    int gm0 = group * G;
    int gsz = min(G, tiles_m - gm0);
    int rem = L - group * G * tiles_n;
    int tm = gm0 + rem % gsz, tn = rem / gsz;
    const int m0 = tm * BM, n0 = tn * BN;

    const int kg = KG > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8) : 0;
    const int tid = threadIdx.x & (kThreads - 1), lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    char *gsm = smem + kg * 2 * STAGE;

    const T *A = (const T *)d.A;
    const T *B = (const T *)d.B;
    const bool avec = (d.lda % VEC) == 0 && ((uintptr_t)A & 15) == 0 && (TA == 1 || (d.K % VEC) == 0);
    const bool bvec = (d.ldb % VEC) == 0 && ((uintptr_t)B & 15) == 0 && (TB == 1 || (d.K % VEC) == 0);

    Loader<T, BM, TA> la;
    Loader<T, BN, TB> lb;
    constexpr bool ILP2 = sizeof(T) == 4 && FM * FN == 1;   // second accumulator bank, see Mfma::mma2
    floatx16 acc[FM][FN], acc2[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = acc2[i][j] = (floatx16){};

    // K is shared by the gridDim.y workgroups of a tile (split-K) and the KG groups of each: group
    // (blockIdx.y, kg) contracts chunks [(blockIdx.y*KG + kg)*nkg, ... + nkg)
    const int nsplit = gridDim.y, split = blockIdx.y;
    const int nk = (d.K + BK - 1) / BK;
    const int nkg = (nk + KG * nsplit - 1) / (KG * nsplit);   // chunks per group
    const int kbeg = (split * KG + kg) * nkg * BK;            // this group's first k (may lie past K: zeros)
    la.load(A, d.lda, m0, d.M, kbeg, d.K, avec, tid);
    lb.load(B, d.ldb, n0, d.N, kbeg, d.K, bvec, tid);
    la.store(gsm, tid);
    lb.store(gsm + BM * 128, tid);
    __syncthreads();

    for (int kt = 0; kt < nkg; kt++) {
        char *cur = gsm + (kt & 1) * STAGE;
        char *nxt = gsm + ((kt + 1) & 1) * STAGE;
        const bool more = kt + 1 < nkg;
        if (more) {
            la.load(A, d.lda, m0, d.M, kbeg + (kt + 1) * BK, d.K, avec, tid);
            lb.load(B, d.ldb, n0, d.N, kbeg + (kt + 1) * BK, d.K, bvec, tid);
        }
        const char *sa = cur, *sb = cur + BM * 128;
        // Fragments are double-buffered: the LDS reads of chunk s+1 are issued before the MFMAs of
        // chunk s, so their latency hides behind those MFMAs.
        vec_t a[2][FM], b[2][FN];
#pragma unroll
        for (int i = 0; i < FM; i++) a[0][i] = *(const vec_t *)(sa + lds_off(wm0 + i * 32 + (lane & 31), lane >> 5));
#pragma unroll
        for (int j = 0; j < FN; j++) b[0][j] = *(const vec_t *)(sb + lds_off(wn0 + j * 32 + (lane & 31), lane >> 5));
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int cb = s & 1, nb = cb ^ 1;
            if (s + 1 < 4) {
                const int c = 2 * (s + 1) + (lane >> 5);
#pragma unroll
                for (int i = 0; i < FM; i++) a[nb][i] = *(const vec_t *)(sa + lds_off(wm0 + i * 32 + (lane & 31), c));
#pragma unroll
                for (int j = 0; j < FN; j++) b[nb][j] = *(const vec_t *)(sb + lds_off(wn0 + j * 32 + (lane & 31), c));
            }
            __builtin_amdgcn_sched_barrier(0);   // keep the next reads ahead of this chunk's MFMAs
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    if constexpr (ILP2) MF::mma2(a[cb][i], b[cb][j], acc[i][j], acc2[i][j]);
                    else MF::mma(a[cb][i], b[cb][j], acc[i][j]);
                }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (more) {
            la.store(nxt, tid);
            lb.store(nxt + BM * 128, tid);
        }
        __syncthreads();
    }

    if constexpr (ILP2) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[i][j] += acc2[i][j];
    }
    if constexpr (KG > 1) {
        // groups 1..KG-1 -> LDS -> group 0, element e of lane l of wave w at [g-1][w][e][l]
        constexpr int NE = FM * FN * 16;
        if (kg > 0) {
            float *red = (float *)smem + ((kg - 1) * 4 + wave) * NE * 64 + lane;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) red[((i * FN + j) * 16 + r) * 64] = acc[i][j][r];
        }
        __syncthreads();
        if (kg == 0)
            for (int g = 1; g < KG; g++) {
                const float *red = (const float *)smem + ((g - 1) * 4 + wave) * NE * 64 + lane;
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[i][j][r] += red[((i * FN + j) * 16 + r) * 64];
            }
    }
    if (nsplit > 1) {
        // Split-K finish. Every split stores group 0's accumulators as its partial with 16-byte buffer
        // stores and the sc1 cache policy (written through, so coherent across the XCDs' L2s), waits
        // for them, and then takes a ticket from the tile's arrival counter; the split that draws the
        // last ticket reads the others' partials the same way (sc1 loads miss in L2), adds all of them
        // in split order (its own from registers, so the sum does not depend on the arrival order),
        // resets the counter for the next launch and runs the epilogue. No workgroup waits on another.
        // Partial layout: 16-byte chunk c of thread t at byte 16 * (c * kThreads + t) of its split.
        constexpr int NC = FM * FN * 4;               // 16-byte chunks per thread
        constexpr int PART = NC * kThreads * 16;      // bytes per split
        constexpr int SC1 = 16;                       // cache policy bit sc1
        typedef unsigned u4 __attribute__((ext_vector_type(4)));
        const int tile = tm * tiles_n + tn;
        int *const count = d.sk_sync + 2 * tile;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            d.sk_part + (long)tile * nsplit * (PART / 4), (short)0, nsplit * PART, 0x00020000);
        __shared__ int ticket;
        if (kg == 0) {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const floatx16 &a = acc[c / (FN * 4)][(c / 4) % FN];
                const int e = (c % 4) * 4;
                const floatx4 v = {a[e], a[e + 1], a[e + 2], a[e + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, split * PART + (c * kThreads + tid) * 16, 0, SC1);
                // wait states before the store's data registers may be rewritten (the compiler has
                // placed such a VALU write two instructions behind a 16-byte store, and it reached memory)
                __builtin_amdgcn_sched_barrier(0);
                asm volatile("s_nop 4" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's partial has landed
        }
        __syncthreads();
        if (threadIdx.x == 0) ticket = ticket_take(count);
        __syncthreads();
        if (ticket != nsplit - 1 || kg > 0) return;
        // every other split stored its partial before taking its ticket; add them in split order, one
        // 32x32 block (4 chunks per split in flight) at a time
#pragma unroll
        for (int bl = 0; bl < FM * FN; bl++) {
            floatx16 &a = acc[bl / FN][bl % FN];
            floatx4 sum[4];
            for (int q = 0; q < nsplit; q++) {
                floatx4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    if (q == split) v[u] = (floatx4){a[4 * u], a[4 * u + 1], a[4 * u + 2], a[4 * u + 3]};
                    else v[u] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, q * PART + ((bl * 4 + u) * kThreads + tid) * 16, 0, SC1));
                }
#pragma unroll
                for (int u = 0; u < 4; u++) sum[u] = q == 0 ? v[u] : sum[u] + v[u];
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int x = 0; x < 4; x++) a[4 * u + x] = sum[u][x];
        }
        if (threadIdx.x == 0) __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // next launch
    }
    if (kg > 0) return;
    epilogue_tile<EPI, T, FM, FN>(d, acc, m0 + wm0, n0 + wn0, lane);
}

template <typename T, int BM, int TA, int TB, int EPI>
static hipError_t launch_t(const GemmDesc &d, hipStream_t s) {
    const int tiles = ((d.M + BM - 1) / BM) * ((d.N + BM - 1) / BM);
    constexpr int VEC = 16 / sizeof(T), BK = 8 * VEC;
    const int nk = (d.K + BK - 1) / BK;
    // Each k-group of a tile (4 waves) runs a register-staged K loop whose iterations wait on their
    // global loads, so short-output, long-K contractions are latency bound on few waves. The automatic
    // choice gives such shapes more wave sets on each tile: k-groups (within one workgroup, up to the
    // tile's LDS budget: 64-tile 4 groups, 128-tile 2) and then splits of K across workgroups (partials
    // folded by the last split to arrive), doubling either while the tile's wave sets stay within 1024
    // (four per CU) and each set keeps at least 2 K chunks.
    int kg = 1, split = 1;
    const bool ws = d.sk_sync && d.sk_part && tiles <= kSplitKMaxTiles;
    if (d.kgroups > 0 && gemm32_kgroups_ok(BM, d.kgroups)) {
        kg = d.kgroups;   // fixed by the caller (a tuner candidate)
    } else {
        const int maxkg = BM == 64 ? 4 : BM == 128 ? 2 : 1;
        while (kg < maxkg && (long)tiles * kg * 2 <= 1024 && nk >= 2 * kg * 2) kg *= 2;
    }
    if (ws && d.splits > 1) {
        split = d.splits > 16 ? 16 : d.splits;   // fixed by the caller (a tuner candidate)
        while (split > 1 && (long)tiles * split * BM * BM > d.sk_cap) split >>= 1;
    } else if (ws && d.splits == 0 && d.kgroups == 0) {
        while (split < 16 && (long)tiles * kg * split * 2 <= 1024 && nk >= 2 * kg * split * 2 &&
               (long)tiles * split * 2 * BM * BM <= d.sk_cap)
            split *= 2;
    }
    const dim3 grid(tiles, split);
    if constexpr (BM == 64) {
        if (kg == 4) { hipLaunchKernelGGL((gemm_kernel<T, BM, BM, TA, TB, EPI, 4>), grid, dim3(kThreads * 4), 0, s, d); return hipGetLastError(); }
    }
    if constexpr (BM <= 128) {
        if (kg == 2) { hipLaunchKernelGGL((gemm_kernel<T, BM, BM, TA, TB, EPI, 2>), grid, dim3(kThreads * 2), 0, s, d); return hipGetLastError(); }
    }
    hipLaunchKernelGGL((gemm_kernel<T, BM, BM, TA, TB, EPI, 1>), grid, dim3(kThreads), 0, s, d);
    return hipGetLastError();
}

template <typename T, int TA, int TB, int EPI>
static hipError_t launch_tile(const GemmDesc &d, hipStream_t s) {
    int tile = d.tile;
    if (tile == 0) {
        long t256 = (long)((d.M + 255) / 256) * ((d.N + 255) / 256);
        long t128 = (long)((d.M + 127) / 128) * ((d.N + 127) / 128);
        tile = t256 >= 224 ? 256 : (t128 >= 192 ? 128 : 64);
    }
    switch (tile) {
        case 256: return launch_t<T, 256, TA, TB, EPI>(d, s);
        case 128: return launch_t<T, 128, TA, TB, EPI>(d, s);
        default: return launch_t<T, 64, TA, TB, EPI>(d, s);
    }
}

template <typename T, int TA, int TB>
static hipError_t launch_epi(const GemmDesc &d, hipStream_t s) {
    switch (d.epi) {
        case EPI_STORE: return launch_tile<T, TA, TB, EPI_STORE>(d, s);
        case EPI_BIAS: return launch_tile<T, TA, TB, EPI_BIAS>(d, s);
        case EPI_BIAS_RELU: return launch_tile<T, TA, TB, EPI_BIAS_RELU>(d, s);
        case EPI_MSE:
            if constexpr (sizeof(T) == 2) return launch_tile<T, TA, TB, EPI_MSE>(d, s);
            else return hipErrorInvalidValue;
        case EPI_MASK: return launch_tile<T, TA, TB, EPI_MASK>(d, s);
        case EPI_SGD: return launch_tile<T, TA, TB, EPI_SGD>(d, s);
        default: return hipErrorInvalidValue;
    }
}

// ── few outputs, long K: one wave per output element ────────────────────────
// Contractions whose M*N outputs are too few to occupy the CUs as tiles (config 1's 64x10 logits,
// config 2's 32x10 fc, config 4's single-row batches) reduce each dot product across the 64 lanes of
// a wave instead: lanes stride K in 16-byte chunks (A and B both K-contiguous), a shuffle tree sums
// them, and lane 0 applies the same scalar epilogue as the tiled kernels.
template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_dot_kernel(GemmDesc d) {
    constexpr int VEC = 16 / sizeof(T);
    const int lane = threadIdx.x & 63;
    const long o = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= (long)d.M * d.N) return;
    const int m = (int)(o / d.N), n = (int)(o % d.N);
    const T *a = (const T *)d.A + (long)m * d.lda, *b = (const T *)d.B + (long)n * d.ldb;
    const bool vec = ((d.lda | d.ldb) % VEC) == 0 && (((uintptr_t)d.A | (uintptr_t)d.B) & 15) == 0;
    float acc = 0.0f;
    int k = lane * VEC;
    if (vec) {
        for (; k + VEC <= d.K; k += 64 * VEC) {
            typedef T vt __attribute__((ext_vector_type(VEC)));
            const vt x = *(const vt *)(a + k), y = *(const vt *)(b + k);
#pragma unroll
            for (int e = 0; e < VEC; e++) acc += (float)x[e] * (float)y[e];
        }
    }
    for (; k < d.K; k += 64 * VEC)
        for (int e = 0; e < VEC && k + e < d.K; e++) acc += (float)a[k + e] * (float)b[k + e];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane != 0) return;
    float in = 0.0f, bias = 0.0f, lossp = 0.0f;
    if constexpr (EPI == EPI_SGD) in = d.W32[(long)m * d.ldc + n];
    if constexpr (EPI == EPI_MASK || EPI == EPI_MSE) in = (float)((const T *)d.aux)[(long)m * d.ldaux + n];
    if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RELU || EPI == EPI_MSE) bias = (float)((const T *)d.bias)[n];
    const float cs = epi_apply<EPI, T>(d, m, n, acc, in, bias, lossp);
    // One wave per output: the partial-sum layouts (GemmDesc::colsum_ld / loss_ld) are filled with
    // atomics here, as 32 waves share each row-block cell (this path serves only small outputs).
    if (d.colsum) atomicAdd(d.colsum + (d.colsum_ld ? (long)(m / 32) * d.colsum_ld : 0) + n, cs);
    if constexpr (EPI == EPI_MSE) atomicAdd(d.lossacc + (d.loss_ld ? (long)(m / 32) * d.loss_ld + n / 32 : 0), lossp);
}

template <typename T>
static hipError_t launch_dot(const GemmDesc &d, hipStream_t s) {
    const long outs = (long)d.M * d.N;
    const dim3 grid((unsigned)((outs + 3) / 4));
    switch (d.epi) {
        case EPI_STORE: hipLaunchKernelGGL((gemm_dot_kernel<T, EPI_STORE>), grid, dim3(256), 0, s, d); break;
        case EPI_BIAS: hipLaunchKernelGGL((gemm_dot_kernel<T, EPI_BIAS>), grid, dim3(256), 0, s, d); break;
        case EPI_BIAS_RELU: hipLaunchKernelGGL((gemm_dot_kernel<T, EPI_BIAS_RELU>), grid, dim3(256), 0, s, d); break;
        case EPI_MSE:
            if constexpr (sizeof(T) == 2) { hipLaunchKernelGGL((gemm_dot_kernel<T, EPI_MSE>), grid, dim3(256), 0, s, d); break; }
            else return hipErrorInvalidValue;
        case EPI_MASK: hipLaunchKernelGGL((gemm_dot_kernel<T, EPI_MASK>), grid, dim3(256), 0, s, d); break;
        case EPI_SGD: hipLaunchKernelGGL((gemm_dot_kernel<T, EPI_SGD>), grid, dim3(256), 0, s, d); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// The dot path takes A and B K-contiguous, at most 16384 outputs and K of at least 256 (where a tile
// would run a long serial K loop on a handful of workgroups).
static bool use_dot(const GemmDesc &d) {
    return d.ta == 0 && d.tb == 0 && d.tile == 0 && (long)d.M * d.N <= 16384 && d.K >= 256;
}

template <typename T>
static hipError_t launch_layout(const GemmDesc &d, hipStream_t s) {
    if (use_dot(d)) return launch_dot<T>(d, s);
    int code = d.ta * 2 + d.tb;
    switch (code) {
        case 0: return launch_epi<T, 0, 0>(d, s);
        case 1: return launch_epi<T, 0, 1>(d, s);
        case 2: return launch_epi<T, 1, 0>(d, s);
        default: return launch_epi<T, 1, 1>(d, s);
    }
}

hipError_t gemm_launch(const GemmDesc &d, hipStream_t s) {
    if (d.M <= 0 || d.N <= 0) return hipSuccess;
    if (d.K < 0) return hipErrorInvalidValue;
    if (d.dtype == GEMM_F16) {
        hipError_t e = hipSuccess;
        if (gemm16_try_launch(d, s, &e)) return e;
        if (d.A2) return hipErrorInvalidValue;   // two-plane contractions run on the direct-to-LDS kernels only
        return launch_layout<half_t>(d, s);
    }
    if (d.A2 || d.C2) return hipErrorInvalidValue;
    // The automatic f32 choice: the direct-to-LDS kernel on 64-wide tiles when they fill the chip, or half
    // of it at K <= 1024 (every 64-wide configuration adds K in the same order, so tuning among them never
    // changes a result), with deeper stages for long K; otherwise the register-staged kernel, whose
    // k-groups and splits of K spread a long K over more waves.
    const long t64 = (long)((d.M + 63) / 64) * ((d.N + 63) / 64);
    if (d.dtype == GEMM_F32 && d.tile == 0 && d.kgroups == 0 && d.splits == 0 && !use_dot(d) &&
        (t64 >= 256 || (t64 >= 128 && d.K <= 1024))) {
        const int cfg = kGemm32dBase + (d.K >= 4096 ? 0 : 2);
        int bm, bk, ns;
        if (gemm32d_config(cfg, &bm, &bk, &ns) && gemm32d_ok(d, bm, bk)) {
            GemmDesc a = d;
            a.tile = cfg;
            return gemm32d_launch(a, s);
        }
    }
    if (d.dtype == GEMM_F32 && d.tile >= kGemm32dBase) {
        int bm, bk, ns;
        if (gemm32d_config(d.tile, &bm, &bk, &ns) && gemm32d_ok(d, bm, bk)) return gemm32d_launch(d, s);
        GemmDesc a = d;   // not a shape this configuration takes: the automatic choice
        a.tile = a.kgroups = a.splits = 0;
        return gemm_launch(a, s);
    }
    if (d.dtype == GEMM_F32) return launch_layout<float>(d, s);
    return hipErrorInvalidValue;
}

}  // namespace ah
