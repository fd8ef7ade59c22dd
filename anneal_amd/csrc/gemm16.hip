// gemm16.hip — f16 MFMA contraction for gfx950 with direct global->LDS loads (no register staging).
//
// Block tile BM x BN (256x256 or 128x128), 4 wave64s in a 2x2 arrangement, K in stages of 64.
// Every operand tile is fetched with global_load_lds_dwordx4 (each lane's 16 bytes land at
// LDS base + 16*lane), so loads for stage k+1 are in flight while stage k is contracted, and no VGPRs
// or ds_write instructions are spent on staging. The layouts are chosen so that the fetch order
// produces a bank-conflict-free LDS image (the LDS of gfx950 has 64 four-byte banks):
//   K-contiguous operand ([rows][K]): two 128-byte rows form a 256-byte super-row whose 16-byte
//     slots are XOR-swizzled by the super-row index; fragments are read with ds_read_b128.
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
constexpr int BK = 64;

// Byte offset of (row r, 16-byte chunk c) in a K-contiguous tile.
__device__ __forceinline__ int koff(int r, int c) {
    const int q = r >> 1;
    return q * 256 + (((((r & 1) << 3) | c) ^ (q & 15)) << 4);
}

// Byte offset of element (k-row k, column m) in an MN-contiguous tile of R columns.
template <int R>
__device__ __forceinline__ int mnoff(int k, int m) {
    return k * (R * 2) + (((m >> 4) ^ ((k & 3) << 1)) << 5) + ((m & 15) << 1);
}

// Per-lane global byte offsets for the 1 KiB blocks this wave fetches (stage-independent part).
template <int R, int T>
struct Fetch {
    static constexpr int NB = R / 8;          // 1 KiB blocks per tile
    static constexpr int PER = NB / 4;        // blocks per wave
    uint32_t off[PER];
    __device__ __forceinline__ void init(long ld, int r0, int rmax, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int b = wave * PER + j;
            if constexpr (T == 0) {
                const int q = 4 * b + (lane >> 4);
                const int x = (lane & 15) ^ (q & 15);
                const int row = min(r0 + 2 * q + (x >> 3), rmax - 1);
                off[j] = (uint32_t)(((long)row * ld + (x & 7) * 8) * 2);
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
    // Issue this wave's loads of stage k0 into `tile` (a 1 KiB-aligned LDS region).
    __device__ __forceinline__ void issue(const char *base, long ld, int k0, char *tile, int wave) const {
        const long adv = T == 0 ? (long)k0 * 2 : (long)k0 * ld * 2;
#pragma unroll
        for (int j = 0; j < PER; j++)
            __builtin_amdgcn_global_load_lds((const void *)(base + adv + off[j]), (void *)(tile + (wave * PER + j) * 1024),
                                             16, 0, 0);
    }
};

template <int R, int T>
__device__ __forceinline__ h8 frag(const char *tile, int r, int s, int lane) {
    if constexpr (T == 0) {
        return *(const h8 *)(tile + koff(r + (lane & 31), 2 * s + (lane >> 5)));
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
template <int BM, int BN, int TA, int TB, int EPI, bool VEPI>
__global__ __launch_bounds__(kThreads) void gemm16_kernel(GemmDesc d) {
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
    constexpr int ABYTES = BM * 128, BBYTES = BN * 128, STAGE = ABYTES + BBYTES;
    __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];
    static_assert(4 * WM * 256 <= 2 * STAGE, "epilogue staging must fit the operand LDS");

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

    Fetch<BM, TA> fa;
    Fetch<BN, TB> fb;
    fa.init(d.lda, m0, d.M, wave, lane);
    fb.init(d.ldb, n0, d.N, wave, lane);
    const char *Ab = (const char *)d.A, *Bb = (const char *)d.B;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = (floatx16){};

    const int nk = d.K / BK;
    fa.issue(Ab, d.lda, 0, smem, wave);
    fb.issue(Bb, d.ldb, 0, smem + ABYTES, wave);
    for (int kt = 0; kt < nk; kt++) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        char *cur = smem + (kt & 1) * STAGE;
        if (kt + 1 < nk) {
            char *nxt = smem + ((kt + 1) & 1) * STAGE;
            fa.issue(Ab, d.lda, (kt + 1) * BK, nxt, wave);
            fb.issue(Bb, d.ldb, (kt + 1) * BK, nxt + ABYTES, wave);
        }
        const char *sa = cur, *sb = cur + ABYTES;
        h8 a[2][FM], b[2][FN];
#pragma unroll
        for (int i = 0; i < FM; i++) a[0][i] = frag<BM, TA>(sa, wm0 + i * 32, 0, lane);
#pragma unroll
        for (int j = 0; j < FN; j++) b[0][j] = frag<BN, TB>(sb, wn0 + j * 32, 0, lane);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int c = s & 1, n = c ^ 1;
            if (s < 3) {
#pragma unroll
                for (int i = 0; i < FM; i++) a[n][i] = frag<BM, TA>(sa, wm0 + i * 32, s + 1, lane);
#pragma unroll
                for (int j = 0; j < FN; j++) b[n][j] = frag<BN, TB>(sb, wn0 + j * 32, s + 1, lane);
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c][i], b[c][j], acc[i][j], 0, 0, 0);
        }
    }

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
    if (vepi) hipLaunchKernelGGL((gemm16_kernel<BM, BM, TA, TB, EPI, true>), dim3(tiles), dim3(kThreads), 0, s, d);
    else hipLaunchKernelGGL((gemm16_kernel<BM, BM, TA, TB, EPI, false>), dim3(tiles), dim3(kThreads), 0, s, d);
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
    if (d.dtype != GEMM_F16 || d.K <= 0 || d.K % BK) return false;
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
