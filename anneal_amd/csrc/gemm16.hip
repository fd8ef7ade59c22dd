// gemm16.hip — f16 MFMA contraction for gfx950 with direct global->LDS loads (no register staging).
//
// Block tile BM x BN (256x256 or 128x128), 4 wave64s in a 2x2 arrangement, K in LDS stages of 32 or 64
// with 4 stages in flight.
// Every operand tile is fetched with global_load_lds_dwordx4 (each lane's 16 bytes land at
// LDS base + 16*lane), so loads for stage k+1 are in flight while stage k is contracted, and no VGPRs
// or ds_write instructions are spent on staging. The layouts are chosen so that the fetch order
// produces a bank-conflict-free LDS image (the LDS of gfx950 has 64 four-byte banks):
//   K-contiguous operand ([rows][K]): rows of 64 or 128 bytes are packed into 256-byte super-rows
//     whose 16-byte slots are XOR-swizzled by the super-row index; fragments are ds_read_b128.
//   MN-contiguous operand ([K][rows]): k-rows stay in the stored orientation, 32-byte segments
//     XOR-swizzled by 2*(k & 3); fragments are read with two ds_read_b64_tr_b16, the CDNA4 LDS
//     transpose read (within 16 lanes, lane j addressing T[kb + j/4][mb + 4*(j%4)] receives
//     T[kb..kb+3][mb + j]), so transposed operands cost no extra pass and no register shuffles.
// Fragments of k-step s+1 are read while the MFMAs of k-step s run. Accumulation is f32
// (codegen/lower.go:667-716 accumulates f16 reduces in f32); f16 products are exact in f32.
#include "ah_common.h"
#include "gemm.h"
#include "gemm_epi.h"

namespace ah {
namespace g16 {

typedef half_t h8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;

constexpr int kThreads = 256;

// Byte offset of (row r, 16-byte chunk c) in a K-contiguous tile whose rows hold BK halves:
// 256-byte super-rows of 256/(2*BK) rows, 16-byte slots XOR-swizzled by the super-row index.
template <int BK>
__device__ __forceinline__ int koff(int r, int c) {
    constexpr int CH = BK / 8, SR = 16 / CH;        // chunks per row, rows per super-row
    const int q = r / SR;
    return q * 256 + ((((r % SR) * CH + c) ^ (q & 15)) << 4);
}

// Byte offset of element (k-row k, column m) in an MN-contiguous tile of R columns.
template <int R>
__device__ __forceinline__ int mnoff(int k, int m) {
    return k * (R * 2) + (((m >> 4) ^ ((k & 3) << 1)) << 5) + ((m & 15) << 1);
}

// Per-lane global byte offsets for the 1 KiB blocks this wave fetches (stage-independent part).
template <int R, int T, int BK>
struct Fetch {
    static constexpr int NB = R * BK * 2 / 1024;   // 1 KiB blocks per tile
    static constexpr int PER = NB / 4;             // blocks per wave
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
                const int seg = (pos16 >> 1) ^ ((kk & 3) << 1);
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
};

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

// VEPI: every wave tile is in bounds and the epilogue arrays admit vector access, so the LDS-staged
// vector epilogue is used (chosen on the host; a kernel holding both epilogues spills registers).
// BK: k per LDS stage (32 or 64); NS: LDS stages in flight (the fetch of stage k+NS-1 is issued
// while stage k is contracted).
template <int BM, int BN, int TA, int TB, int EPI, bool VEPI, int BK, int NS>
__global__ __launch_bounds__(kThreads) void gemm16_kernel(GemmDesc d) {
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
    constexpr int ABYTES = BM * BK * 2, BBYTES = BN * BK * 2, STAGE = ABYTES + BBYTES;
    constexpr int KS = BK / 16;                                           // MFMA k-steps per stage
    constexpr int PERSTAGE = Fetch<BM, TA, BK>::PER + Fetch<BN, TB, BK>::PER;
    constexpr int SMEM = (NS * STAGE > 4 * WM * 256) ? NS * STAGE : 4 * WM * 256;
    __shared__ __attribute__((aligned(1024))) char smem[SMEM];

    const int tiles_n = (d.N + BN - 1) / BN;
    const int tiles_m = (d.M + BM - 1) / BM;
    const int ntiles = tiles_m * tiles_n;
    int L = blockIdx.x;
    if ((ntiles & 7) == 0) L = (L & 7) * (ntiles >> 3) + (L >> 3);   // contiguous tile runs per XCD
    constexpr int G = 4;
    const int group = L / (G * tiles_n);
    const int gm0 = group * G;
    const int gsz = min(G, tiles_m - gm0);
    const int rem = L - group * G * tiles_n;
    const int m0 = (gm0 + rem % gsz) * BM, n0 = (rem / gsz) * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;

    Fetch<BM, TA, BK> fa;
    Fetch<BN, TB, BK> fb;
    fa.init(d.lda, m0, d.M, wave, lane);
    fb.init(d.ldb, n0, d.N, wave, lane);
    const char *Ab = (const char *)d.A, *Bb = (const char *)d.B;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = (floatx16){};

    const int nk = d.K / BK;
#pragma unroll
    for (int p = 0; p < NS - 1; p++) {
        const int kp = min(p, nk - 1) * BK;
        fa.issue(Ab, d.lda, kp, smem + p * STAGE, wave);
        fb.issue(Bb, d.ldb, kp, smem + p * STAGE + ABYTES, wave);
    }
    for (int kt = 0; kt < nk; kt++) {
        // stage kt has landed once at most the NS-2 younger stages are still in flight
#ifndef AH_EXP_NOBARRIER
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NS - 2) * PERSTAGE) : "memory");
        __syncthreads();
#endif
        const char *sa = smem + (kt % NS) * STAGE, *sb = sa + ABYTES;
        // Refill the buffer consumed in the previous iteration with stage kt+NS-1 (clamped: the
        // tail re-fetches the last stage into idle buffers, keeping the loop one basic block).
        char *nxt = smem + ((kt + NS - 1) % NS) * STAGE;
        const int kn = min(kt + NS - 1, nk - 1) * BK;
        h8 a[2][FM], b[2][FN];
#pragma unroll
        for (int i = 0; i < FM; i++) a[0][i] = frag<BM, TA, BK>(sa, wm0 + i * 32, 0, lane);
#pragma unroll
        for (int j = 0; j < FN; j++) b[0][j] = frag<BN, TB, BK>(sb, wn0 + j * 32, 0, lane);
        // Scheduling fences fix the issue order: the LDS reads of k-step s+1 go out as a group ahead
        // of the MFMAs of k-step s (their latency hides behind the MFMAs); the stage fetches are
        // spread evenly between the MFMAs (issued back to back they fill the vector-memory queue
        // and stall MFMA issue); MFMAs of different k-steps, which share accumulators, never mix.
        __builtin_amdgcn_sched_barrier(0);
        constexpr int NM = FM * FN;
        constexpr int PA = Fetch<BM, TA, BK>::PER;
        constexpr int FPS = (PERSTAGE + KS - 1) / KS;                      // fetches per k-step
        // Spreading pays on the 256x256 tile (16 MFMAs per k-step); on 128x128 (4 per k-step) the
        // fences cost more than they hide, so its fetches go out as one group.
        constexpr bool SPREAD = NM >= 16;
        if constexpr (!SPREAD) {
#ifndef AH_EXP_NOFETCH
            fa.issue(Ab, d.lda, kn, nxt, wave);
            fb.issue(Bb, d.ldb, kn, nxt + ABYTES, wave);
#endif
        }
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const int c = s & 1, n = c ^ 1;
            if (s + 1 < KS) {
#pragma unroll
                for (int i = 0; i < FM; i++) a[n][i] = frag<BM, TA, BK>(sa, wm0 + i * 32, s + 1, lane);
#pragma unroll
                for (int j = 0; j < FN; j++) b[n][j] = frag<BN, TB, BK>(sb, wn0 + j * 32, s + 1, lane);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int t = 0; t < NM; t++) {
                acc[t / FN][t % FN] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c][t / FN], b[c][t % FN], acc[t / FN][t % FN], 0, 0, 0);
                if (SPREAD && t % (NM / FPS) == NM / FPS - 1) {
                    const int f = s * FPS + t / (NM / FPS);
#ifndef AH_EXP_NOFETCH
                    if (f < PA) fa.issue_one(f, Ab, d.lda, kn, nxt, wave);
                    else if (f < PERSTAGE) fb.issue_one(f - PA, Bb, d.ldb, kn, nxt + ABYTES, wave);
#endif
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // drain the tail re-fetches before LDS reuse

    const int mb = m0 + wm0, nb = n0 + wn0;
    if constexpr (VEPI) {
        // Epilogue through the (now idle) operand LDS: each wave owns FM*32 rows x 64 f32 columns.
        __syncthreads();
        epilogue_lds<EPI, half_t, FM, FN>(d, acc, mb, nb, lane, smem + wave * (WM * 256));
    } else {
        epilogue_tile<EPI, half_t, FM, FN>(d, acc, mb, nb, lane);
    }
}

template <int T>
static bool operand_ok(const void *p, long ld, int rows) {
    if (((uintptr_t)p & 15) || (ld % 8) || rows < 8) return false;
    return T == 0 || (rows % 8) == 0;
}

template <int BM, int TA, int TB, int EPI>
static hipError_t launch(const GemmDesc &d, hipStream_t s) {
    int tiles = ((d.M + BM - 1) / BM) * ((d.N + BM - 1) / BM);
    const uintptr_t a = (uintptr_t)d.C | (uintptr_t)d.aux | (uintptr_t)d.bias | (uintptr_t)d.W32 |
                        (uintptr_t)d.W16 | (uintptr_t)d.gout;
    const bool vepi = d.M % BM == 0 && d.N % BM == 0 && d.ldc % 4 == 0 && d.ldaux % 4 == 0 && (a & 15) == 0;
    // k=64 per stage, 2 stages (256x256: 128 KiB; 128x128: 64 KiB). Deeper pipelines with k=32
    // stages measured slower: each stage ends in a workgroup barrier, and halving the stage doubles them.
    constexpr int BK = 64;
    constexpr int NS = 2;
    if (vepi) hipLaunchKernelGGL((gemm16_kernel<BM, BM, TA, TB, EPI, true, BK, NS>), dim3(tiles), dim3(kThreads), 0, s, d);
    else hipLaunchKernelGGL((gemm16_kernel<BM, BM, TA, TB, EPI, false, BK, NS>), dim3(tiles), dim3(kThreads), 0, s, d);
    return hipGetLastError();
}

template <int TA, int TB, int EPI>
static hipError_t launch_tile(const GemmDesc &d, hipStream_t s) {
    int tile = d.tile;
    if (tile == 0) {
        long t256 = (long)((d.M + 255) / 256) * ((d.N + 255) / 256);
        tile = t256 >= 224 ? 256 : 128;
    }
    return tile == 256 ? launch<256, TA, TB, EPI>(d, s) : launch<128, TA, TB, EPI>(d, s);
}

template <int TA, int TB>
static hipError_t launch_epi(const GemmDesc &d, hipStream_t s) {
    switch (d.epi) {
        case EPI_STORE: return launch_tile<TA, TB, EPI_STORE>(d, s);
        case EPI_BIAS: return launch_tile<TA, TB, EPI_BIAS>(d, s);
        case EPI_BIAS_RELU: return launch_tile<TA, TB, EPI_BIAS_RELU>(d, s);
        case EPI_MSE: return launch_tile<TA, TB, EPI_MSE>(d, s);
        case EPI_MASK: return launch_tile<TA, TB, EPI_MASK>(d, s);
        case EPI_SGD: return launch_tile<TA, TB, EPI_SGD>(d, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace g16

// Returns true (and launches) when the shape/alignment admits the direct-to-LDS f16 kernel.
bool gemm16_try_launch(const GemmDesc &d, hipStream_t s, hipError_t *err) {
    using namespace g16;
    if (d.dtype != GEMM_F16 || d.K <= 0 || d.K % 64) return false;
    if (d.tile != 0 && d.tile != 128 && d.tile != 256) return false;
    bool ok = (d.ta ? operand_ok<1>(d.A, d.lda, d.M) : operand_ok<0>(d.A, d.lda, d.M)) &&
              (d.tb ? operand_ok<1>(d.B, d.ldb, d.N) : operand_ok<0>(d.B, d.ldb, d.N));
    if (!ok) return false;
    switch (d.ta * 2 + d.tb) {
        case 0: *err = launch_epi<0, 0>(d, s); break;
        case 1: *err = launch_epi<0, 1>(d, s); break;
        case 2: *err = launch_epi<1, 0>(d, s); break;
        default: *err = launch_epi<1, 1>(d, s); break;
    }
    return true;
}

}  // namespace ah
