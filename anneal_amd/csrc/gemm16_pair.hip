// gemm16_pair.hip — two independent f16 contractions in one launch, the first split over K.
//
// The config-3 backward has two pairs of contractions that read only finished inputs and write
// disjoint outputs: dW3 beside dH1, and dW1 beside dW2. The 1024-wide weight gradients alone fill a
// quarter of the 256 CUs with 256x256 tiles (64 tiles, 64 k-stages each). In a paired launch the first
// contraction's tiles are split over K into `nsplit` parts (a workgroup each, folded by G16Split below)
// and come first in the grid, so 64 x 4 = 256 short workgroups fill the chip at once; the
// second contraction's 256 tiles follow as workgroups free their CUs. Every CU then runs one quarter
// tile and one whole tile, one launch replaces two, and the first contraction's epilogue overlaps the
// second's main loops. Compiled once per variant (-DAH_G16_PV=<n>, a 256x256 single-k-group variant).
#include "gemm16_kernel.h"

#ifndef AH_G16_PV
#error "compile with -DAH_G16_PV=<variant>"
#endif

namespace ah {
namespace g16 {

// Split of K over the workgroups of one output tile. Each split stores its f32 partial tile with
// 16-byte buffer stores and the sc1 cache policy (the policy of device-scope atomic stores: written
// through to memory, so coherent across the XCDs' L2s), waits for them, and then takes a ticket from
// the tile's arrival counter; the split that draws the last ticket reads the others' partials the same
// way (sc1 loads miss in L2), adds all of them in split order (its own from registers, so the sum does
// not depend on the arrival order), resets the counter for the next launch and runs the epilogue. No
// workgroup ever waits on another. Partial layout: 16-byte chunk c of lane t at byte 16 * (c * NT + t).
struct G16Split {
    int split, nsplit;   // this workgroup's split, splits per tile
    int *count;          // the tile's arrival counter (zero before the launch, zero after it)
    float *part;         // the tile's nsplit partial tiles, NT * FM * FN * 16 floats each
    int *ticket;         // an LDS word for broadcasting the ticket
    template <int FM, int FN, int NT>
    __device__ __forceinline__ bool run(floatx16 (&acc)[FM][FN], int tid) const {
        constexpr int NC = FM * FN * 4;                    // 16-byte chunks per lane
        constexpr int PART = NC * NT * 16;                 // bytes per partial
        constexpr int SC1 = 16;                            // cache policy bit sc1
        typedef unsigned u4 __attribute__((ext_vector_type(4)));
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(part, (short)0, nsplit * PART, 0x00020000);
        const int own = split * PART + tid * 16;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const floatx16 &a = acc[c / (FN * 4)][(c / 4) % FN];
            const int e = (c % 4) * 4;
            const floatx4 v = {a[e], a[e + 1], a[e + 2], a[e + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, own + c * NT * 16, 0, SC1);
            // wait states before the store's data registers may be rewritten (the compiler once placed
            // such a VALU write two instructions behind a 16-byte store, and it reached the memory)
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_nop 4" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's partial has landed
        __syncthreads();
        if (threadIdx.x == 0) *ticket = ticket_take(count);
        __syncthreads();
        if (*ticket != nsplit - 1) return false;
        // every other split stored its partial before taking its ticket; add them in split order,
        // one 32x32 block at a time (4 chunks per split in flight)
#pragma unroll
        for (int b = 0; b < FM * FN; b++) {
            floatx4 sum[4];
            for (int q = 0; q < nsplit; q++) {
                floatx4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int c = b * 4 + u;
                    const floatx16 &a = acc[b / FN][b % FN];
                    if (q == split) v[u] = (floatx4){a[4 * u], a[4 * u + 1], a[4 * u + 2], a[4 * u + 3]};
                    else v[u] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, q * PART + tid * 16 + c * NT * 16, 0, SC1));
                }
#pragma unroll
                for (int u = 0; u < 4; u++) sum[u] = q == 0 ? v[u] : sum[u] + v[u];
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int x = 0; x < 4; x++) acc[b / FN][b % FN][4 * u + x] = sum[u][x];
        }
        if (threadIdx.x == 0) __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }
};

template <int V, int TA0, int TB0, int EPI0, int TA1, int TB1, int EPI1>
__global__ __launch_bounds__(64 * Var<V>::WVM * Var<V>::WVN) void gemm16_pair_kernel(G16PairArgs p) {
    using P = Var<V>;
    constexpr int BM = P::BM;
    static_assert(P::KG == 1, "paired launches use single-k-group variants");
    __shared__ __attribute__((aligned(1024))) char smem[G16Smem<BM, BM, P::BK, P::NS, P::WVM, P::WVN, P::FETCH, 1>::SMEM];
    __shared__ int ticket;
    int L = blockIdx.x;
    if (L < p.items0) {
        const int tm = p.d0.M / BM, tn = p.d0.N / BM, tiles = tm * tn;
        if ((p.items0 & 7) == 0) L = (L & 7) * (p.items0 >> 3) + (L >> 3);   // contiguous runs per XCD
        // split-major: the workgroups of one XCD contract the same k range of neighbouring tiles
        const int split = L / tiles, t = L - split * tiles;
        int m0, n0;
        g16_tile_origin(t, tm, tn, BM, BM, m0, n0);
        const int klen = p.d0.K / p.nsplit;
        g16_tile<BM, BM, TA0, TB0, EPI0, true, P::BK, P::NS, P::WVM, P::WVN, P::FETCH, P::XB, 1>(
            p.d0, smem, m0, n0, (long)split * klen, klen,
            G16Split{split, p.nsplit, p.count + t, p.part + (long)t * p.nsplit * BM * BM, &ticket});
    } else {
        L -= p.items0;
        const int tm = p.d1.M / BM, tn = p.d1.N / BM, tiles = tm * tn;
        if ((tiles & 7) == 0) L = (L & 7) * (tiles >> 3) + (L >> 3);
        int m0, n0;
        g16_tile_origin(L, tm, tn, BM, BM, m0, n0);
        g16_tile<BM, BM, TA1, TB1, EPI1, true, P::BK, P::NS, P::WVM, P::WVN, P::FETCH, P::XB, 1>(
            p.d1, smem, m0, n0, 0, p.d1.K, G16NoFold{});
    }
}

template <int TA0, int TB0, int EPI0, int TA1, int TB1, int EPI1>
static hipError_t launch_pair(const G16PairArgs &p, int items1, hipStream_t s) {
    constexpr int V = AH_G16_PV;
    hipLaunchKernelGGL((gemm16_pair_kernel<V, TA0, TB0, EPI0, TA1, TB1, EPI1>), dim3(p.items0 + items1),
                       dim3(64 * Var<V>::WVM * Var<V>::WVN), 0, s, p);
    return hipGetLastError();
}

}  // namespace g16

#define AH_G16P_NAME2(n) gemm16_pair_variant_##n
#define AH_G16P_NAME(n) AH_G16P_NAME2(n)

// The layout/epilogue combinations instantiated: (weight gradient, SGD) beside (weight gradient,
// SGD) or beside (input gradient, ReLU mask); a split forward contraction with the MSE epilogue alone.
hipError_t AH_G16P_NAME(AH_G16_PV)(const G16PairArgs &p, int items1, bool *supported, hipStream_t s) {
    using namespace g16;
    const GemmDesc &a = p.d0, &b = p.d1;
    *supported = true;
    const int ka = a.ta * 2 + a.tb, kb = b.ta * 2 + b.tb;
    if (ka == 3 && a.epi == EPI_SGD) {
        if (items1 == 0 || (kb == 3 && b.epi == EPI_SGD)) return launch_pair<1, 1, EPI_SGD, 1, 1, EPI_SGD>(p, items1, s);
        if (kb == 1 && b.epi == EPI_MASK) return launch_pair<1, 1, EPI_SGD, 0, 1, EPI_MASK>(p, items1, s);
    }
    if (ka == 0 && a.epi == EPI_MSE && items1 == 0) return launch_pair<0, 0, EPI_MSE, 0, 0, EPI_MSE>(p, 0, s);
    *supported = false;
    return hipSuccess;
}

}  // namespace ah
