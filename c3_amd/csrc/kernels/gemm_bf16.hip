// gemm_bf16.hip -- bf16 GEMMs of the fused Linear(+bias)(+ReLU) layer on
// gfx950 bf16 MFMA (v_mfma_f32_32x32x16_bf16), fp32 accumulation.
//
// Same three GEMMs and fusions as gemm_f32.hip (forward with bias+act
// epilogue; dX and dW with the ReLU mask applied while the dY tile is loaded;
// db as a side output of dW).  The reference has no bf16 path (every kernel
// body is f32, include/C3/Graph.h:43); this is the reduced-precision variant
// of the same arithmetic: bf16 storage, fp32 accumulate, bias and activation
// in fp32, one round-to-nearest-even on the bf16 outputs.
//
// LDS holds both operands as [row][k] with k contiguous (row = m for A, n
// for B), 64 k per stage, rows padded to 72 elements (144 bytes) so that the
// 16-byte fragment reads of 8 consecutive lanes cover all banks once.
// An operand whose k index is contiguous in global memory is copied as is;
// one whose rows are contiguous (W in the forward, X^T and dY in dW) is read
// as 8x8 blocks (8 k-rows of 8 consecutive row elements) and transposed in
// registers before the LDS store.
//
// MFMA 32x32x16: lane l supplies 8 bf16 of row l%32 at k = 16s + 8(l/32) .. +7
// for step s, for A and B alike, so every output sums the full k range.
// Accumulator layout as in the fp32 kernel: lane l, register v -> row
// 8*(v/4) + 4*(l/32) + v%4, column l%32 of the 32x32 block.
#include "gemm_common.h"

namespace {

constexpr int kBK = 64;       // k depth of one LDS stage
constexpr int kStride = 72;   // bf16 elements per LDS row (64 + 8 padding)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// bf16 bits: Y > 0 <=> sign clear, nonzero, not NaN (+inf counts as > 0).
__device__ __forceinline__ bool bf16_gt0(unsigned short y) { return (short)y > 0 && y <= 0x7f80u; }

// (Y > 0 ? 1 : 0) * dY on bf16 bit patterns: dY when Y > 0, else a zero with
// dY's sign, or NaN when dY is Inf/NaN (0 * Inf = NaN).
__device__ __forceinline__ unsigned short bf16_mask_mul(unsigned short y, unsigned short d) {
    if (bf16_gt0(y)) return d;
    if ((d & 0x7f80u) == 0x7f80u) return 0x7fc0u;
    return d & 0x8000u;
}

__device__ __forceinline__ uint32_t mask_mul2(uint32_t y, uint32_t d) {
    return (uint32_t)bf16_mask_mul((unsigned short)(y & 0xffff), (unsigned short)(d & 0xffff)) |
           ((uint32_t)bf16_mask_mul((unsigned short)(y >> 16), (unsigned short)(d >> 16)) << 16);
}

__device__ __forceinline__ u32x4 mask_mul8(u32x4 y, u32x4 d) {
    return u32x4{mask_mul2(y[0], d[0]), mask_mul2(y[1], d[1]), mask_mul2(y[2], d[2]), mask_mul2(y[3], d[3])};
}

// Global -> register -> LDS staging of one ROWS x 64 operand tile.
template <int ROWS, int NT, bool KC, bool MASK>
struct Bf16Loader {
    // KC: ROWS*8 vectors of 8 k-values; vector v -> row v/8, k 8*(v%8).
    // !KC: ROWS units of 8x8; unit u -> k-block u%8, row-block u/8.
    static constexpr int UNITS = KC ? ROWS * 8 : ROWS;
    static constexpr int NV = (UNITS + NT - 1) / NT;
    static_assert(UNITS % NT == 0 || UNITS < NT, "tile must split evenly over the block");
    static constexpr int NREG = KC ? NV : NV * 8;

    u32x4 r[NREG];
    uint32_t off0;  // element offset of this thread's first vector at k-tile 0
    int rr0, kk0;   // tile-relative row / k of that vector

    // KC: vector v -> row v/8, k 8*(v%8); rows step NT/8 per i.
    // !KC: unit u -> k-block u%8, row-block u/8; row blocks step NT/8 per i.
    __device__ __forceinline__ void init(int tid, int64_t ld, int64_t grow0) {
        if (KC) {
            rr0 = tid >> 3;
            kk0 = 8 * (tid & 7);
            off0 = (uint32_t)((grow0 + rr0) * ld + kk0);
        } else {
            kk0 = 8 * (tid & 7);
            rr0 = 8 * (tid >> 3);
            off0 = (uint32_t)(kk0 * ld + grow0 + rr0);
        }
    }

    // P advanced to the tile's k0 (KC: P + k0; !KC: P + k0*ld).
    __device__ __forceinline__ void load(const unsigned short* __restrict__ P, const unsigned short* __restrict__ Pm,
                                         uint32_t ld, int64_t rows_left, int64_t k_left, int tid) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int u = tid + NT * i;
            if (UNITS < NT && u >= UNITS) break;
            if (KC) {
                const int rr = rr0 + i * (NT / 8);
                const uint32_t off = off0 + (uint32_t)(i * (NT / 8)) * ld;
                u32x4 x = {0u, 0u, 0u, 0u};
                if (rr < rows_left && kk0 < k_left) {
                    x = *(const u32x4*)(P + off);
                    if (MASK) x = mask_mul8(*(const u32x4*)(Pm + off), x);
                }
                r[i] = x;
            } else {
                const int rr = rr0 + i * NT;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const uint32_t off = off0 + (uint32_t)(i * NT) + (uint32_t)q * ld;
                    u32x4 x = {0u, 0u, 0u, 0u};
                    if (rr < rows_left && kk0 + q < k_left) {
                        x = *(const u32x4*)(P + off);
                        if (MASK) x = mask_mul8(*(const u32x4*)(Pm + off), x);
                    }
                    r[8 * i + q] = x;
                }
            }
        }
    }

    __device__ __forceinline__ void store(unsigned short* __restrict__ S, int tid) const {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int u = tid + NT * i;
            if (UNITS < NT && u >= UNITS) break;
            if (KC) {
                const int rr = rr0 + i * (NT / 8);
                *(u32x4*)(S + rr * kStride + kk0) = r[i];
            } else {
                const int rr = rr0 + i * NT;
                // r[8i + q] holds k-row kk0+q, elements rows rr..rr+7 (2 per dword).
                // Output c: row rr+c, k kk0..kk0+7 (2 per dword).
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const int d = c >> 1;
                    u32x4 w;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t lo = r[8 * i + 2 * j][d], hi = r[8 * i + 2 * j + 1][d];
                        w[j] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
                    }
                    *(u32x4*)(S + (rr + c) * kStride + kk0) = w;
                }
            }
        }
    }
};

template <int BM, int BN, int WAVES_M, int WAVES_N, bool AK, bool BKC, bool AMASK, bool BMASK, bool DB,
          bool OUT_BF16>
__device__ __forceinline__ void gemm_bf16_body(const GemmArgs& p) {
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int A_SIZE = BM * kStride, B_SIZE = BN * kStride;
    constexpr int STAGE = A_SIZE + B_SIZE;
    static_assert(FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tile of 32x32 blocks");

    __shared__ __attribute__((aligned(16))) unsigned short smem[2 * STAGE];
    __shared__ float db_part[DB ? NT : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn;
    tile_coords<8>(p.M, p.N, BM, BN, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const unsigned short* __restrict__ A = (const unsigned short*)p.A;
    const unsigned short* __restrict__ Am = (const unsigned short*)p.Amask;
    const unsigned short* __restrict__ B = (const unsigned short*)p.B;
    const unsigned short* __restrict__ Bm = (const unsigned short*)p.Bmask;

    Bf16Loader<BM, NT, AK, AMASK> la;
    Bf16Loader<BN, NT, BKC, BMASK> lb;
    la.init(tid, p.lda, m0);
    lb.init(tid, p.ldb, n0);
    const int64_t a_rows = p.M - m0, b_rows = p.N - n0;
    const uint32_t lda = (uint32_t)p.lda, ldb = (uint32_t)p.ldb;
    const int64_t a_kstep = AK ? kBK : (int64_t)kBK * p.lda;
    const int64_t b_kstep = BKC ? kBK : (int64_t)kBK * p.ldb;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const bool do_db = DB && p.db != nullptr && tm == 0;
    float dbacc = 0.0f;

    const int nk = (int)((p.K + kBK - 1) / kBK);
    la.load(A, Am, lda, a_rows, p.K, tid);
    lb.load(B, Bm, ldb, b_rows, p.K, tid);
    la.store(smem, tid);
    lb.store(smem + A_SIZE, tid);
    __syncthreads();

    const int r = lane & 31, g = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const unsigned short* As = smem + cur * STAGE;
        const unsigned short* Bs = As + A_SIZE;
        const bool more = kt + 1 < nk;
        if (more) {
            const int64_t k0 = (int64_t)(kt + 1) * kBK;
            const int64_t ao = (int64_t)(kt + 1) * a_kstep, bo = (int64_t)(kt + 1) * b_kstep;
            la.load(A + ao, AMASK ? Am + ao : Am, lda, a_rows, p.K - k0, tid);
            lb.load(B + bo, BMASK ? Bm + bo : Bm, ldb, b_rows, p.K - k0, tid);
        }

#pragma unroll
        for (int s = 0; s < kBK / 16; ++s) {
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *(const bf16x8*)(As + (wm * TM + 32 * i + r) * kStride + 16 * s + 8 * g);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bfr[j] = *(const bf16x8*)(Bs + (wn * TN + 32 * j + r) * kStride + 16 * s + 8 * g);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }

        if (DB && do_db) {
            // Row c of the B tile is column c of dZ: thread (c, part) sums its k-slice.
            static_assert(!DB || NT % BN == 0, "threads per column");
            constexpr int RPT = NT / BN, KPT = kBK / RPT;
            const int c = tid % BN, part = tid / BN;
#pragma unroll
            for (int k = 0; k < KPT; ++k) dbacc += bf16_to_f32(Bs[c * kStride + part * KPT + k]);
        }

        if (more) {
            unsigned short* Ns = smem + (cur ^ 1) * STAGE;
            la.store(Ns, tid);
            lb.store(Ns + A_SIZE, tid);
        }
        __syncthreads();
    }

    if (DB && do_db) {
        constexpr int RPT = NT / BN;
        db_part[tid] = dbacc;
        __syncthreads();
        if (tid < BN) {
            float s = 0.0f;
#pragma unroll
            for (int q = 0; q < RPT; ++q) s += db_part[tid + q * BN];
            const int64_t n = n0 + tid;
            if (n < p.N) p.db[n] = s;
        }
    }

#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t n = n0 + wn * TN + 32 * j + r;
        const bool nok = n < p.N;
        const float bv = (p.bias != nullptr && nok) ? p.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t m = m0 + wm * TM + 32 * i + 8 * (v >> 2) + 4 * g + (v & 3);
                if (nok && m < p.M) {
                    float x = acc[i][j][v];
                    if (p.bias != nullptr) x = x + bv;
                    x = act_apply(x, p.act);
                    if (OUT_BF16)
                        ((unsigned short*)p.C)[m * p.ldc + n] = f32_to_bf16_rne(x);
                    else
                        ((float*)p.C)[m * p.ldc + n] = x;
                }
            }
        }
    }
}

}  // namespace

#define C3_GEMM_BF16_ONE(NAME, BM, BN, WM, WN, AK, BKC, AMASK, BMASK, DB, OUTB)                       \
    extern "C" __global__ __launch_bounds__(64 * WM * WN) void NAME(GemmArgs p) {                    \
        gemm_bf16_body<BM, BN, WM, WN, AK, BKC, AMASK, BMASK, DB, OUTB>(p);                          \
    }

// Kinds as in gemm_f32.hip.  Forward and dX write bf16; dW writes fp32.
// Plain matmul (c3hip_matmul with bf16) writes bf16 for every transpose case.
#define C3_GEMM_BF16_KINDS(T, BM, BN, WM, WN)                                                          \
    C3_GEMM_BF16_ONE(c3_gemm_bf16_fwd_##T, BM, BN, WM, WN, true, false, false, false, false, true)     \
    C3_GEMM_BF16_ONE(c3_gemm_bf16_dx_##T, BM, BN, WM, WN, true, true, false, false, false, true)       \
    C3_GEMM_BF16_ONE(c3_gemm_bf16_dx_mask_##T, BM, BN, WM, WN, true, true, true, false, false, true)   \
    C3_GEMM_BF16_ONE(c3_gemm_bf16_dw_##T, BM, BN, WM, WN, false, false, false, false, true, false)     \
    C3_GEMM_BF16_ONE(c3_gemm_bf16_dw_mask_##T, BM, BN, WM, WN, false, false, false, true, true, false) \
    C3_GEMM_BF16_ONE(c3_gemm_bf16_dwb_##T, BM, BN, WM, WN, false, false, false, false, false, true)    \
    C3_GEMM_BF16_ONE(c3_gemm_bf16_tt_##T, BM, BN, WM, WN, false, true, false, false, false, true)

C3_GEMM_BF16_KINDS(t64x64, 64, 64, 2, 2)
C3_GEMM_BF16_KINDS(t128x128, 128, 128, 2, 2)
C3_GEMM_BF16_KINDS(t256x128, 256, 128, 2, 2)
C3_GEMM_BF16_KINDS(t256x256, 256, 256, 2, 2)
