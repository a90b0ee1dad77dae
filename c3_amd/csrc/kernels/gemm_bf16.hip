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

    with_act(p.act, [&](auto at) {
        constexpr int ACT = decltype(at)::value;
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
                        x = act_c<ACT>(x);
                        if (OUT_BF16)
                            ((unsigned short*)p.C)[m * p.ldc + n] = f32_to_bf16_rne(x);
                        else
                            ((float*)p.C)[m * p.ldc + n] = x;
                    }
                }
            }
        }
    });
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

// ===========================================================================
// Direct-to-LDS kernels: 256x256 block tiles (8 waves of 128x64, 4 waves of
// 128x128, or 8 ping-pong waves), 128x128 tiles (4 waves of 64x64) or 64x64
// tiles (4 waves of 32x32), BK-deep k tiles in STAGES LDS stages.
// Global tiles go straight into LDS with global_load_lds_dwordx4 (lane l's
// 16 bytes land at base + 16*l of the instruction's 1 KiB), so no staging
// registers and no LDS stores are needed.  Layouts, per operand:
//   KC (k contiguous in global): LDS [row][BK k], BK/8 16-byte chunks per
//     row; chunk c of row r sits in slot c ^ s(r), s(r) = (r >> 1) & 7 for
//     BK = 64 and (r >> 2) & 3 for BK = 32.  Measured on MI355X (64 LDS
//     banks): these are the XOR keys under which the 32 rows one
//     ds_read_b128 fragment read touches fall into distinct banks; keying on
//     r & 7 leaves a 2-way conflict.  Fragment: one ds_read_b128.
//   RC (row contiguous in global): LDS [BK k][ROWS], the chunk holding rows
//     8c..8c+7 of k-row kr sits in slot c ^ (4 * (kr % 4)) (64-row tiles:
//     c ^ (4 * ((kr / 2) % 2)), see rc_key).  A k-row of a 256-row tile is
//     512 bytes, so every k-row starts on bank 0; the 32 lanes of one half of
//     a transposed read address k-rows kbase..kbase+3 and chunks c0..c0+3,
//     and the key 4 * (kr % 4) puts those 16 (kr, c) pairs on 16 distinct
//     16-byte bank groups (no conflict; the key 2 * (kr % 4) left a 2-way
//     conflict, 2 extra cycles per read in the LDS counters).  Fragment: two
//     ds_read_b64_tr_b16; in each 16-lane group lane j receives element j%4
//     of the 8-byte pieces addressed by lanes 4r + j/4 (r = 0..3), so lanes
//     address k-rows kbase + (j/4) at column offset 4*(j%4) and each lane
//     gets 4 consecutive k of its own row (column).
// Pipeline: tiles kt+1 .. kt+STAGES-1 are in flight while tile kt is
// multiplied.  Each wave issues the same number of DMA instructions per tile,
// so "tile kt has landed" is s_waitcnt vmcnt(<instructions issued after it>);
// the barrier that follows makes every wave's part of tile kt visible and
// ends every read of the stage that is refilled next.
// Requires the contiguous extents % 8 == 0 (host-checked); K % BK == 0 for
// the ping-pong and 4-wave kernels, any K for the others (a partial last
// k-tile, DirectTile::issue_partial); rows past M or N are loaded from a
// clamped address and never stored.
// ===========================================================================
namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int ROWS, bool KC, int NWAVES, int BK>
struct DirectTile {
    static constexpr int BYTES = ROWS * BK * 2;
    static constexpr int NI = BYTES / 1024 / NWAVES;  // 1 KiB load instructions per wave per tile
    static constexpr int KC_CPR = BK / 8;             // KC: 16-byte chunks per row
    static constexpr int RC_CPR = ROWS / 8;           // RC: 16-byte chunks per k-row
    static_assert(BYTES % (1024 * NWAVES) == 0, "tile must split into whole instructions per wave");
    static_assert(BK == 32 || BK == 64, "BK is 32 or 64");
    static_assert(KC || ROWS == 64 || ROWS >= 128, "RC swizzle keys are for 8 or >= 16 chunks per k-row");
    uint32_t goff[NI];

    __device__ __forceinline__ static int kc_key(int r) { return BK == 64 ? ((r >> 1) & 7) : ((r >> 2) & 3); }
    // RC: k-rows of >= 256 bytes start on bank 0 (key 4 (kr % 4) over 16
    // chunks); 128-byte k-rows (ROWS = 64) put two k-rows on each 256-byte
    // bank row, so k-rows kr and kr + 1 already differ by 8 bank groups and
    // the key 4 ((kr / 2) % 2) over 8 chunks separates kr from kr + 2.
    __device__ __forceinline__ static int rc_key(int kr) { return ROWS >= 128 ? 4 * (kr & 3) : 4 * ((kr >> 1) & 1); }

    // grow0: first global row (m or n) of the tile; rows_total bounds it.
    __device__ __forceinline__ void init(int wave, int lane, int64_t ld, int64_t grow0, int64_t rows_total) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int q = wave * NI + i;
            if (KC) {
                const int r = (64 / KC_CPR) * q + lane / KC_CPR;
                const int c = (lane % KC_CPR) ^ kc_key(r);
                int64_t gr = grow0 + r;
                if (gr > rows_total - 1) gr = rows_total - 1;
                goff[i] = (uint32_t)(gr * ld + 8 * c);
            } else {
                const int kr = q * (64 / RC_CPR) + lane / RC_CPR;
                const int c = (lane % RC_CPR) ^ rc_key(kr);
                int64_t gc = grow0 + 8 * c;
                if (gc > rows_total - 8) gc = rows_total - 8;
                goff[i] = (uint32_t)(kr * ld + gc);
            }
        }
    }

    // P advanced to the k-tile (KC: + k0, RC: + k0*ld); S = this operand's LDS tile.
    // The loads are issued through inline asm (M0 = LDS destination of the
    // instruction, wave-uniform): the compiler then does not treat them as
    // LDS writes that every later LDS read must wait for; the kernel orders
    // them itself with s_waitcnt vmcnt and barriers.
    __device__ __forceinline__ void issue(const unsigned short* P, unsigned short* S, int wave) const {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(S + (wave * NI + i) * 512);
            const unsigned short* src = P + goff[i];
            asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                         :
                         : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(src)
                         : "memory", "m0");
        }
    }

    // issue() with the operand tile's LDS byte address given (computed once
    // per kernel instead of converting a generic pointer per instruction).
    __device__ __forceinline__ void issue_lds(const unsigned short* P, uint32_t s_lds, int wave) const {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t lds = s_lds + (uint32_t)((wave * NI + i) * 1024);
            const unsigned short* src = P + goff[i];
            asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                         :
                         : "s"(lds), "v"(src)
                         : "memory", "m0");
        }
    }

    // A last k-tile holding only kr < BK valid k (kr a multiple of 8 for KC
    // operands, any for RC ones): lanes whose 16-byte chunk lies below kr
    // issue their DMA as issue() does; the others write zeros to the LDS slot
    // their DMA would fill, so the fragments past kr are exact zeros and
    // nothing beyond the operand is read.  A wave may skip DMA instructions
    // here, so every tile wait from the issue of this tile on is vmcnt(0)
    // (the kernels' counted waits assume NI instructions per tile).
    __device__ __forceinline__ void issue_partial(const unsigned short* P, unsigned short* S, int wave, int lane,
                                                  int kr) const {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int q = wave * NI + i;
            // KC: the lane's global chunk is its LDS slot XOR the row's key
            // (see init); RC: its k-row.
            const int kc_row = (64 / KC_CPR) * q + lane / KC_CPR;
            const bool valid = KC ? (8 * ((lane % KC_CPR) ^ kc_key(kc_row)) < kr)
                                  : (q * (64 / RC_CPR) + lane / RC_CPR < kr);
            unsigned short* slot = S + q * 512;
            if (valid) {
                const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)slot;
                const unsigned short* src = P + goff[i];
                asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                             :
                             : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(src)
                             : "memory", "m0");
            } else {
                *(u32x4*)(slot + 8 * lane) = u32x4{0u, 0u, 0u, 0u};
            }
        }
    }

    // The i-th of this wave's NI DMA instructions (same effect as issue() for
    // that instruction alone), so the issue can be spread between MFMAs.
    __device__ __forceinline__ void issue_one(const unsigned short* P, unsigned short* S, int wave, int i) const {
        const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(S + (wave * NI + i) * 512);
        const unsigned short* src = P + goff[i];
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                     :
                     : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(src)
                     : "memory", "m0");
    }

    // 8 bf16 (k = 16*st + 8*(lane/32) .. +7) of tile row r0 + lane%32.
    __device__ __forceinline__ static bf16x8 frag(const unsigned short* S, int r0, int st, int lane) {
        if (KC) {
            const int row = r0 + (lane & 31);
            const int slot = (2 * st + (lane >> 5)) ^ kc_key(row);
            return *(const bf16x8*)(S + row * BK + slot * 8);
        } else {
            const int G = lane >> 4, sp = lane & 15;
            const int col = r0 + 16 * (G & 1) + 4 * (sp & 3);
            s16x4 v[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int kr = 16 * st + 8 * (G >> 1) + 4 * h + (sp >> 2);
                const int slot = (col >> 3) ^ rc_key(kr);
                v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(S + kr * ROWS + slot * 8 + (col & 7)));
            }
            i16x8 w = {v[0][0], v[0][1], v[0][2], v[0][3], v[1][0], v[1][1], v[1][2], v[1][3]};
            return __builtin_bit_cast(bf16x8, w);
        }
    }
};

// s_waitcnt vmcnt(n) alone (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait until at most min(after, J) tiles' DMA instructions (NIW per tile)
// are outstanding.
template <int NIW, int J>
__device__ __forceinline__ void wait_tiles_upto(int after) {
    if constexpr (J == 0) {
        wait_vmcnt<0>();
    } else {
        if (after >= J) wait_vmcnt<J * NIW>();
        else wait_tiles_upto<NIW, J - 1>(after);
    }
}

// Wait until at most `after` (< PF) tiles' DMA instructions are outstanding.
template <int NIW, int PF>
__device__ __forceinline__ void wait_tiles_after(int after) {
    wait_tiles_upto<NIW, PF - 1>(after);
}

// Epilogue of the direct kernels.  Their MFMAs take the B fragment as the
// first operand, so each 32x32 accumulator block holds C transposed: lane l,
// register v of block (i, q) is C[mb + 32i + l%32][nb + 32q + 8(v/4) +
// 4(l/32) + v%4], four consecutive columns per register group.  fp32 output
// stores those 16 bytes as they are; bf16 output packs them to 8 bytes and
// v_permlane32_swap trades halves between lanes l and l + 32 so that each
// lane holds 8 consecutive columns (16 bytes): lanes 0..31 columns 8t..8t+7,
// lanes 32..63 columns 8(t+1).., for t = 0, 2.  Every store then moves 16
// bytes per lane.  Columns past N and rows past M are never written; a tile
// edge, an unaligned C or a leading dimension that breaks 16-byte alignment
// takes the element-wise path.
// EPI: 0 store bf16, 1 bias + act then store bf16, 2 store fp32.
// One 32x32 block: a = its accumulators, m = this lane's row, nq = the
// block's first column, bv = the bias of this lane's 16 columns.
template <int EPI, int ACT>
__device__ __forceinline__ void store_block_t(const GemmArgs& p, const f32x16& a, int64_t m, int64_t nq,
                                              const float (&bv)[16], bool vec, int h) {
    float x[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        x[v] = a[v];
        if (EPI == 1) {
            if (p.bias != nullptr) x[v] = x[v] + bv[v];
            x[v] = act_c<ACT>(x[v]);
        }
    }
    if (EPI == 2) {
        float* C = (float*)p.C + m * p.ldc;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int64_t n0 = nq + 8 * t + 4 * h;
            if (m < p.M) {
                if (vec && n0 + 4 <= p.N) {
                    *(f32x4*)(C + n0) = f32x4{x[4 * t], x[4 * t + 1], x[4 * t + 2], x[4 * t + 3]};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n0 + e < p.N) C[n0 + e] = x[4 * t + e];
                }
            }
        }
    } else {
        uint32_t P[4][2];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int d = 0; d < 2; ++d)
                P[t][d] = (uint32_t)f32_to_bf16_rne(x[4 * t + 2 * d]) |
                          ((uint32_t)f32_to_bf16_rne(x[4 * t + 2 * d + 1]) << 16);
        unsigned short* C = (unsigned short*)p.C + m * p.ldc;
#pragma unroll
        for (int t = 0; t < 4; t += 2) {
            uint32_t w[4];
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                // Lanes 0..31 keep their own group t and take lane l + 32's;
                // lanes 32..63 take lane l - 32's group t + 1 and keep their own.
                const auto r = __builtin_amdgcn_permlane32_swap(P[t][d], P[t + 1][d], false, false);
                w[d] = r[0];
                w[2 + d] = r[1];
            }
            const int64_t n0 = nq + 8 * (t + h);
            if (m < p.M) {
                if (vec && n0 + 8 <= p.N) {
                    *(u32x4*)(C + n0) = u32x4{w[0], w[1], w[2], w[3]};
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (n0 + e < p.N) C[n0 + e] = (unsigned short)(w[e >> 1] >> (16 * (e & 1)));
                }
            }
        }
    }
}

// Blocks are visited through template recursion so that every accumulator
// index is a constant (a loop the compiler declined to unroll would index
// the array at run time and move it to scratch memory).  Column block q's 16
// bias values are loaded once, before its FM blocks are stored: a load after
// a store to C cannot be moved ahead of it (C might alias the bias), so
// loading them per 32x32 block made every block wait a memory round trip
// (15 us per 256x256 tile).
template <int EPI, int ACT, int FM, int FN, int Q, int I>
__device__ __forceinline__ void store_rows_t(const GemmArgs& p, f32x16 (&acc)[FM][FN], int64_t mb, int64_t nq,
                                             const float (&bv)[16], bool vec, int lane) {
    if constexpr (I < FM) {
        store_block_t<EPI, ACT>(p, acc[I][Q], mb + 32 * I + (lane & 31), nq, bv, vec, lane >> 5);
        store_rows_t<EPI, ACT, FM, FN, Q, I + 1>(p, acc, mb, nq, bv, vec, lane);
    }
}

template <int EPI, int ACT, int FM, int FN, int Q>
__device__ __forceinline__ void store_blocks_t(const GemmArgs& p, f32x16 (&acc)[FM][FN], int64_t mb, int64_t nb,
                                               bool vec, int lane) {
    if constexpr (Q < FN) {
        const int h = lane >> 5;
        const int64_t nq = nb + 32 * Q;
        float bv[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t n = nq + 8 * (v >> 2) + 4 * h + (v & 3);
            bv[v] = (EPI == 1 && p.bias != nullptr && n < p.N) ? p.bias[n] : 0.0f;
        }
        store_rows_t<EPI, ACT, FM, FN, Q, 0>(p, acc, mb, nq, bv, vec, lane);
        store_blocks_t<EPI, ACT, FM, FN, Q + 1>(p, acc, mb, nb, vec, lane);
    }
}

template <int EPI, int FM, int FN>
__device__ __forceinline__ void store_tile_t(const GemmArgs& p, f32x16 (&acc)[FM][FN], int64_t mb, int64_t nb,
                                             int lane) {
    const bool vec = ((uintptr_t)p.C & 15) == 0 && (p.ldc & (EPI == 2 ? 3 : 7)) == 0;
    if (EPI == 1)
        with_act(p.act, [&](auto at) { store_blocks_t<EPI, decltype(at)::value, FM, FN, 0>(p, acc, mb, nb, vec, lane); });
    else
        store_blocks_t<EPI, 0, FM, FN, 0>(p, acc, mb, nb, vec, lane);
}

// bf16 output of a wave's TM x TN tile through LDS (region: TM * TN bf16 of
// the kernel's stages, free once every wave is past its last k-step): each
// lane writes its 4-column groups (the values store_block_t computes, the
// same operations) into a row-major copy whose 16-byte chunks are XOR-keyed
// by row (r & 7), then reads back whole 16-byte chunks so that one store
// instruction writes 8 rows x 128 contiguous bytes instead of 32 rows x 32.
// Only for whole tiles with vector-aligned C (else store_tile_t).
template <int EPI, int ACT, int FM, int FN>
__device__ __forceinline__ void stage_tile_t(const GemmArgs& p, f32x16 (&acc)[FM][FN], int64_t mrow0, int64_t nb,
                                             int lane, unsigned short* region) {
    constexpr int TN = 32 * FN, RB = TN * 2;  // row bytes
    const int h = lane >> 5;
#pragma unroll
    for (int q = 0; q < FN; ++q) {
        const int64_t nq = nb + 32 * q;
        float bv[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t n = nq + 8 * (v >> 2) + 4 * h + (v & 3);
            bv[v] = (EPI == 1 && p.bias != nullptr) ? p.bias[n] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int r = 32 * i + (lane & 31);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float x[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[e] = acc[i][q][4 * t + e];
                    if (EPI == 1) {
                        if (p.bias != nullptr) x[e] = x[e] + bv[4 * t + e];
                        x[e] = act_c<ACT>(x[e]);
                    }
                }
                const uint32_t w0 = (uint32_t)f32_to_bf16_rne(x[0]) | ((uint32_t)f32_to_bf16_rne(x[1]) << 16);
                const uint32_t w1 = (uint32_t)f32_to_bf16_rne(x[2]) | ((uint32_t)f32_to_bf16_rne(x[3]) << 16);
                const int chunk = 4 * q + t;
                char* dst = (char*)region + r * RB + ((chunk ^ (r & 7)) * 16) + h * 8;
                *(uint2*)dst = make_uint2(w0, w1);
            }
        }
    }
    constexpr int CPR = TN / 8, RPI = 64 / CPR;  // chunks per row, rows per instruction
    const int cr = lane / CPR, ck = lane % CPR;
#pragma unroll
    for (int s = 0; s < 32 * FM / RPI; ++s) {
        const int r = RPI * s + cr;
        const u32x4 v = *(const u32x4*)((const char*)region + r * RB + ((ck ^ (r & 7)) * 16));
        *(u32x4*)((unsigned short*)p.C + (mrow0 + r) * p.ldc + nb + 8 * ck) = v;
    }
}

// The LDS stages of a direct kernel: one array per size, so the two GEMM
// bodies of a layer-backward launch (tiles with stages of one size) share it.
template <int ELEMS>
__device__ __forceinline__ unsigned short* direct_smem() {
    __shared__ __attribute__((aligned(1024))) unsigned short smem[ELEMS];
    return smem;
}

// EARLY: after each tile barrier, issue the first k-step's fragment reads
// before the DMA of the next tile (whose inline asm orders memory), with the
// LDS addresses of the stages computed once.  The DMA issue is ~50 scalar
// instructions; issued first, it held every wave's first reads (and so the
// matrix cores of the whole CU) right after each barrier.  Measured on
// MI355X against the plain order, alternating in one process: d256w8 at
// 8192x4096x4096 forward +7% (1026 -> 1096 TF/s), dX +1%, dW +0.3%; at
// 16384x8192x8192 +2% / +3% / +0.5%.  Issuing the last k-step's MFMAs after
// the next tile's barrier as well (so they cover that barrier) was 1-3% slower.
// bid: the block's index among this GEMM's blocks (blockIdx.x by default).
template <int WAVES_M, int WAVES_N, bool AK, bool BKC, int EPI, int BK, int STAGES, int BM, int BN, bool EARLY = false,
          bool STAGED = false>
__device__ __forceinline__ void gemm_bf16_direct_body(const GemmArgs& p, int bid = -1) {
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N, FM = TM / 32, FN = TN / 32;
    constexpr int PF = STAGES - 1;  // tiles in flight ahead of the one multiplied
    using TA = DirectTile<BM, AK, NW, BK>;
    using TB = DirectTile<BN, BKC, NW, BK>;
    constexpr int A_EL = TA::BYTES / 2, B_EL = TB::BYTES / 2, STAGE = A_EL + B_EL;
    constexpr int NIW = TA::NI + TB::NI;
    static_assert(PF * NIW < 64, "outstanding DMA instructions exceed vmcnt");

    unsigned short* const smem = direct_smem<STAGES * STAGE>();

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn;
    tile_coords<8>(p.M, p.N, BM, BN, tm, tn, bid);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const unsigned short* A = (const unsigned short*)p.A;
    const unsigned short* B = (const unsigned short*)p.B;
    TA la;
    TB lb;
    la.init(wave, lane, p.lda, m0, p.M);
    lb.init(wave, lane, p.ldb, n0, p.N);
    const int64_t a_kstep = AK ? BK : (int64_t)BK * p.lda;
    const int64_t b_kstep = BKC ? BK : (int64_t)BK * p.ldb;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // k-tiles; the last one holds kr_last valid k (BK when K % BK == 0).  A
    // partial last tile skips the DMA instructions of its invalid chunks, so
    // once it is issued (from iteration nk - PF on) the waits are vmcnt(0).
    const int nk = (int)((p.K + BK - 1) / BK);
    const int kr_last = (int)(p.K - (int64_t)(nk - 1) * BK);
    const int k_exact_until = kr_last < BK ? nk - PF : nk;
    const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)smem);
    auto issue_tile = [&](int t, int stage) {
        unsigned short* S = smem + stage * STAGE;
        if (t == nk - 1 && kr_last < BK) {
            la.issue_partial(A + (int64_t)t * a_kstep, S, wave, lane, kr_last);
            lb.issue_partial(B + (int64_t)t * b_kstep, S + A_EL, wave, lane, kr_last);
        } else if (EARLY) {
            const uint32_t sl = smem_lds + (uint32_t)(stage * STAGE * 2);
            la.issue_lds(A + (int64_t)t * a_kstep, sl, wave);
            lb.issue_lds(B + (int64_t)t * b_kstep, sl + (uint32_t)(A_EL * 2), wave);
        } else {
            la.issue(A + (int64_t)t * a_kstep, S, wave);
            lb.issue(B + (int64_t)t * b_kstep, S + A_EL, wave);
        }
    };
#pragma unroll
    for (int t = 0; t < PF; ++t) {
        if (t < nk) issue_tile(t, t);
    }

    for (int kt = 0; kt < nk; ++kt) {
        wait_tiles_after<NIW, PF>(kt < k_exact_until ? min(nk - 1 - kt, PF - 1) : 0);
        __syncthreads();
        const unsigned short* As = smem + (kt % STAGES) * STAGE;
        const unsigned short* Bs = As + A_EL;
        bf16x8 af0[FM], bf0[FN];
        if (EARLY) {
#pragma unroll
            for (int i = 0; i < FM; ++i) af0[i] = TA::frag(As, wm * TM + 32 * i, 0, lane);
#pragma unroll
            for (int j = 0; j < FN; ++j) bf0[j] = TB::frag(Bs, wn * TN + 32 * j, 0, lane);
        }
        if (kt + PF < nk) issue_tile(kt + PF, (kt + PF) % STAGES);
#pragma unroll
        for (int st = 0; st < BK / 16; ++st) {
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = (EARLY && st == 0) ? af0[i] : TA::frag(As, wm * TM + 32 * i, st, lane);
#pragma unroll
            for (int j = 0; j < FN; ++j) bfr[j] = (EARLY && st == 0) ? bf0[j] : TB::frag(Bs, wn * TN + 32 * j, st, lane);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
        }
    }

    if constexpr (STAGED && EPI != 2 && TN >= 64) {
        static_assert(NW * TM * TN <= STAGES * STAGE, "staging fits the stages");
        const int64_t mr = m0 + wm * TM, nc = n0 + wn * TN;
        const bool whole = mr + TM <= p.M && nc + TN <= p.N && ((uintptr_t)p.C & 15) == 0 && (p.ldc & 7) == 0;
        if (whole) {
            __syncthreads();  // every wave past its last fragment read
            unsigned short* region = smem + wave * (TM * TN);
            if (EPI == 1)
                with_act(p.act, [&](auto at) { stage_tile_t<EPI, decltype(at)::value, FM, FN>(p, acc, mr, nc, lane, region); });
            else
                stage_tile_t<EPI, 0, FM, FN>(p, acc, mr, nc, lane, region);
            return;
        }
    }
    store_tile_t<EPI, FM, FN>(p, acc, m0 + wm * TM, n0 + wn * TN, lane);
}


// ---------------------------------------------------------------------------
// Interleaved register-pipelined schedule (suffix _rq): 4 waves of 128x128
// (2x2), one per SIMD, each with two fragment sets; BK-deep k tiles in STAGES
// LDS stages, STAGES - 1 tiles in flight ahead of the one multiplied; an
// explicit instruction order.  A wave issues in order, and a run of
// LDS reads (or DMA issues) holds back the MFMAs queued behind it; so each
// MFMA of step s is followed by at most one fragment read of step s + 1 and
// one DMA instruction, and the order is pinned with scheduling barriers.
// Measured on MI355X: issuing a k-step's 12 LDS reads as one run before its
// 16 MFMAs costs about a third of the MFMA rate even when the MFMAs do not
// depend on the reads.  Tile switch: at the last step, wait for the next
// tile's DMA and pass the barrier, then interleave that step's MFMAs with
// the next tile's first reads; the DMA of tile t + STAGES - 1 (into the stage
// tile t - 1 used, free since the barrier that ended tile t - 1) is
// interleaved with tile t's first-step MFMAs.
// ---------------------------------------------------------------------------
template <bool AK, bool BKC, int EPI, int BK, int STAGES>
__device__ __forceinline__ void gemm_bf16_rq_body(const GemmArgs& p) {
    constexpr int BM = 256, BN = 256, NW = 4, PF = STAGES - 1;
    constexpr int FM = 4, FN = 4;  // 128x128 per wave
    constexpr int KSTEPS = BK / 16;
    using TA = DirectTile<BM, AK, NW, BK>;
    using TB = DirectTile<BN, BKC, NW, BK>;
    constexpr int A_EL = TA::BYTES / 2, B_EL = TB::BYTES / 2, STAGE = A_EL + B_EL;
    constexpr int NIW = TA::NI + TB::NI;
    static_assert(NIW <= FM * FN, "DMA instructions are spread one per MFMA");
    static_assert(PF * NIW < 64, "outstanding DMA instructions exceed vmcnt");
    static_assert(KSTEPS % 2 == 0, "fragment sets alternate per step");

    __shared__ __attribute__((aligned(1024))) unsigned short smem[STAGES * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    int tm, tn;
    tile_coords<8>(p.M, p.N, BM, BN, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const unsigned short* A = (const unsigned short*)p.A;
    const unsigned short* B = (const unsigned short*)p.B;
    TA la;
    TB lb;
    la.init(wave, lane, p.lda, m0, p.M);
    lb.init(wave, lane, p.ldb, n0, p.N);
    const int64_t a_kstep = AK ? BK : (int64_t)BK * p.lda;
    const int64_t b_kstep = BKC ? BK : (int64_t)BK * p.ldb;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int nk = (int)(p.K / BK);
    const int r0 = wm * 128, c0 = wn * 128;
    // Tiles 0 .. PF - 1 before the loop; tile t + PF during tile t.
#pragma unroll
    for (int u = 0; u < PF; ++u) {
        if (u < nk) {
            la.issue(A + (int64_t)u * a_kstep, smem + u * STAGE, wave);
            lb.issue(B + (int64_t)u * b_kstep, smem + u * STAGE + A_EL, wave);
        }
    }
    wait_tiles_after<NIW, PF>(min(nk - 1, PF - 1));
    __syncthreads();

    bf16x8 fa[2][FM], fb[2][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) fa[0][i] = TA::frag(smem, r0 + 32 * i, 0, lane);
#pragma unroll
    for (int j = 0; j < FN; ++j) fb[0][j] = TB::frag(smem + A_EL, c0 + 32 * j, 0, lane);

    for (int t = 0; t < nk; ++t) {
        const unsigned short* As = smem + (t % STAGES) * STAGE;
        const bool dma = t + PF < nk;
        const unsigned short* Ag = A + (int64_t)(t + PF) * a_kstep;
        const unsigned short* Bg = B + (int64_t)(t + PF) * b_kstep;
        unsigned short* Sd = smem + ((t + PF) % STAGES) * STAGE;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            const int cur = s & 1, nxt = cur ^ 1;
            const bool last = s + 1 == KSTEPS;
            const bool reads = !last || t + 1 < nk;
            if (last && t + 1 < nk) {
                // Tile t + 1 must have landed (tiles up to t + PF may be in flight).
                wait_tiles_after<NIW, PF>(min(nk - 2 - t, PF - 1));
                __builtin_amdgcn_sched_barrier(0);
                __syncthreads();
                __builtin_amdgcn_sched_barrier(0);
            }
            const unsigned short* Sr = last ? smem + ((t + 1) % STAGES) * STAGE : As;
            const int sr = last ? 0 : s + 1;
#pragma unroll
            for (int q = 0; q < FM * FN; ++q) {
                const int i = q / FN, j = q % FN;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[cur][j], fa[cur][i], acc[i][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (reads && q < FM) fa[nxt][q] = TA::frag(Sr, r0 + 32 * q, sr, lane);
                if (reads && q >= FM && q < FM + FN) fb[nxt][q - FM] = TB::frag(Sr + A_EL, c0 + 32 * (q - FM), sr, lane);
                if (s == 0 && dma && q < NIW) {
                    if (q < TA::NI)
                        la.issue_one(Ag, Sd, wave, q);
                    else
                        lb.issue_one(Bg, Sd + A_EL, wave, q - TA::NI);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    store_tile_t<EPI, FM, FN>(p, acc, m0 + r0, n0 + c0, lane);
}

// ---------------------------------------------------------------------------
// Ping-pong schedule (suffix _pp): 8 waves, two per SIMD (waves w and w + 4
// share SIMD w % 4), each computing a 128x64 part of the 256x256 tile
// (group g = w / 4 takes rows 128g .. 128g + 127, wave w % 4 the columns
// 64(w % 4) ..).  The two groups alternate between a load phase (fragment
// reads of one BK-deep k tile from LDS into registers, plus the group's
// share of the DMA of a later tile) and a compute phase (the MFMAs of the
// fragments loaded in the previous phase), offset by one phase: while the
// waves of one group issue MFMAs the other group's waves on the same SIMDs
// issue LDS traffic, so the matrix core of each SIMD is fed by alternate
// waves and the LDS reads never stand in its issue queue.  Phases end at
// block barriers; group 1 passes one extra barrier at the start and skips
// its last one, so both groups pass the same number.
// Global phase 2j: group 0 loads tile j, group 1 computes tile j - 1;
// phase 2j + 1: group 0 computes tile j, group 1 loads tile j.  Tile t sits
// in stage t % STAGES; its last reader is group 1 in phase 2t + 1, so in
// phase 2j (group 0) and 2j + 1 (group 1) each group issues its share of
// tile j + STAGES - 1 into the stage tile j - 1 held.  Tile j + 1 is first
// read in phase 2j + 2: every wave waits for its own DMA of that tile
// before the barrier that ends phase 2j + 1.
// ---------------------------------------------------------------------------
template <bool AK, bool BKC, int EPI, int BK, int STAGES>
__device__ __forceinline__ void gemm_bf16_pp_body(const GemmArgs& p) {
    constexpr int BM = 256, BN = 256, NW = 8, TM = 128, TN = 64, FM = TM / 32, FN = TN / 32;
    constexpr int KSTEPS = BK / 16;
    using TA = DirectTile<BM, AK, NW, BK>;
    using TB = DirectTile<BN, BKC, NW, BK>;
    constexpr int A_EL = TA::BYTES / 2, B_EL = TB::BYTES / 2, STAGE = A_EL + B_EL;
    constexpr int NIW = TA::NI + TB::NI;
    static_assert(STAGES >= 2 && STAGES <= 4, "2 to 4 stages");
    static_assert((STAGES - 1) * NIW < 64, "outstanding DMA instructions exceed vmcnt");

    __shared__ __attribute__((aligned(1024))) unsigned short smem[STAGES * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;
    const int r0 = grp * TM, c0 = (wave & 3) * TN;

    int tm, tn;
    tile_coords<8>(p.M, p.N, BM, BN, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const unsigned short* A = (const unsigned short*)p.A;
    const unsigned short* B = (const unsigned short*)p.B;
    TA la;
    TB lb;
    la.init(wave, lane, p.lda, m0, p.M);
    lb.init(wave, lane, p.ldb, n0, p.N);
    const int64_t a_kstep = AK ? BK : (int64_t)BK * p.lda;
    const int64_t b_kstep = BKC ? BK : (int64_t)BK * p.ldb;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int nk = (int)(p.K / BK);
#pragma unroll
    for (int u = 0; u < STAGES; ++u) {
        if (u < nk) {
            la.issue(A + (int64_t)u * a_kstep, smem + u * STAGE, wave);
            lb.issue(B + (int64_t)u * b_kstep, smem + u * STAGE + A_EL, wave);
        }
    }
    // Tile 0 landed everywhere (up to STAGES - 1 later tiles may be in flight).
    wait_tiles_after<NIW, STAGES>(min(nk - 1, STAGES - 1));
    __syncthreads();
    if (grp == 1) __syncthreads();

    bf16x8 fa[KSTEPS][FM], fb[KSTEPS][FN];
    for (int j = 0; j < nk; ++j) {
        // Load phase of tile j.
        const unsigned short* As = smem + (j % STAGES) * STAGE;
        if (j >= 1 && j + STAGES - 1 < nk) {
            unsigned short* Sd = smem + ((j + STAGES - 1) % STAGES) * STAGE;
            la.issue(A + (int64_t)(j + STAGES - 1) * a_kstep, Sd, wave);
            lb.issue(B + (int64_t)(j + STAGES - 1) * b_kstep, Sd + A_EL, wave);
        }
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
            for (int i = 0; i < FM; ++i) fa[s][i] = TA::frag(As, r0 + 32 * i, s, lane);
#pragma unroll
            for (int q = 0; q < FN; ++q) fb[s][q] = TB::frag(As + A_EL, c0 + 32 * q, s, lane);
        }
        // Tiles issued so far: up to min(j + STAGES - 1, nk - 1); tile j + 1 must land.
        const int after = min(STAGES - 2, nk - 2 - j);
        if (grp == 1) wait_tiles_after<NIW, STAGES - 1>(max(after, 0));
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        // Compute phase of tile j.
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int q = 0; q < FN; ++q)
                    acc[i][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[s][q], fa[s][i], acc[i][q], 0, 0, 0);
        if (grp == 0) wait_tiles_after<NIW, STAGES - 1>(max(after, 0));
        __builtin_amdgcn_sched_barrier(0);
        if (grp == 0 || j + 1 < nk) __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
    }

    store_tile_t<EPI, FM, FN>(p, acc, m0 + r0, n0 + c0, lane);
}

// Split-K: block row blockIdx.y of the grid multiplies k in [y * split_k,
// y * split_k + split_k) and writes its fp32 partial product to C + y *
// c_split; c3_splitk_reduce adds the partials.  Only fp32-output kinds split.
template <bool AK, bool BKC, int EPI>
__device__ __forceinline__ GemmArgs split_args(const GemmArgs& p) {
    if (EPI != 2 || p.split_k == 0) return p;
    GemmArgs q = p;
    const int64_t k0 = (int64_t)blockIdx.y * p.split_k;
    q.A = (const unsigned short*)p.A + (AK ? k0 : k0 * p.lda);
    q.B = (const unsigned short*)p.B + (BKC ? k0 : k0 * p.ldb);
    q.K = min(p.split_k, p.K - k0);
    q.C = (float*)p.C + (int64_t)blockIdx.y * p.c_split;
    return q;
}

}  // namespace

#define C3_GEMM_BF16_PP(NAME, AK, BKC, EPI, BK, ST) \
    extern "C" __global__ __launch_bounds__(512) void NAME(GemmArgs p) { gemm_bf16_pp_body<AK, BKC, EPI, BK, ST>(split_args<AK, BKC, EPI>(p)); }
#define C3_GEMM_BF16_PP_KINDS(T, BK, ST)                                   \
    C3_GEMM_BF16_PP(c3_gemm_bf16_fwd_##T, true, false, 1, BK, ST)          \
    C3_GEMM_BF16_PP(c3_gemm_bf16_dx_##T, true, true, 0, BK, ST)            \
    C3_GEMM_BF16_PP(c3_gemm_bf16_dw_##T, false, false, 2, BK, ST)          \
    C3_GEMM_BF16_PP(c3_gemm_bf16_dwb_##T, false, false, 0, BK, ST)         \
    C3_GEMM_BF16_PP(c3_gemm_bf16_tt_##T, false, true, 0, BK, ST)          \
    C3_GEMM_BF16_PP(c3_gemm_bf16_fwdt_##T, true, true, 1, BK, ST)         \
    C3_GEMM_BF16_PP(c3_gemm_bf16_fwdf_##T, true, false, 2, BK, ST)        \
    C3_GEMM_BF16_PP(c3_gemm_bf16_dxf_##T, true, true, 2, BK, ST)          \
    C3_GEMM_BF16_PP(c3_gemm_bf16_ttf_##T, false, true, 2, BK, ST)

// d256pp: 32-deep k, 4 stages (128 KiB of LDS).
C3_GEMM_BF16_PP_KINDS(d256pp, 32, 4)

#define C3_GEMM_BF16_D(NAME, WM, WN, AK, BKC, EPI, BK, ST, BT) C3_GEMM_BF16_DE(NAME, WM, WN, AK, BKC, EPI, BK, ST, BT, false)
#define C3_GEMM_BF16_DE(NAME, WM, WN, AK, BKC, EPI, BK, ST, BT, E) C3_GEMM_BF16_DES(NAME, WM, WN, AK, BKC, EPI, BK, ST, BT, E, false)
#define C3_GEMM_BF16_DES(NAME, WM, WN, AK, BKC, EPI, BK, ST, BT, E, SG)                                    \
    extern "C" __global__ __launch_bounds__(64 * WM * WN) void NAME(GemmArgs p) {                         \
        gemm_bf16_direct_body<WM, WN, AK, BKC, EPI, BK, ST, BT, BT, E, SG>(split_args<AK, BKC, EPI>(p));   \
    }

// fwd: X (KC) . W (RC) + bias, act -> bf16.  fwdt: the same with W given
// transposed ([N, K], KC).  dx: dZ (KC) . W^T (KC) -> bf16.
// dw: X^T (RC) . dZ (RC) -> fp32.  dwb: same, bf16 out.  tt: A^T (RC) . B^T (KC) -> bf16.
// FSG: the bf16-output forwards store through LDS (stage_tile_t).
#define C3_GEMM_BF16_D_KINDS(T, WM, WN, BK, ST, BT) C3_GEMM_BF16_D_KINDS_S(T, WM, WN, BK, ST, BT, false)
#define C3_GEMM_BF16_D_KINDS_S(T, WM, WN, BK, ST, BT, FSG)                                 \
    C3_GEMM_BF16_DES(c3_gemm_bf16_fwd_##T, WM, WN, true, false, 1, BK, ST, BT, true, FSG)   \
    C3_GEMM_BF16_DE(c3_gemm_bf16_dx_##T, WM, WN, true, true, 0, BK, ST, BT, true)           \
    C3_GEMM_BF16_DE(c3_gemm_bf16_dw_##T, WM, WN, false, false, 2, BK, ST, BT, true)         \
    C3_GEMM_BF16_DE(c3_gemm_bf16_dwb_##T, WM, WN, false, false, 0, BK, ST, BT, true)        \
    C3_GEMM_BF16_DE(c3_gemm_bf16_tt_##T, WM, WN, false, true, 0, BK, ST, BT, true)          \
    C3_GEMM_BF16_DES(c3_gemm_bf16_fwdt_##T, WM, WN, true, true, 1, BK, ST, BT, true, FSG)   \
    C3_GEMM_BF16_DE(c3_gemm_bf16_fwdf_##T, WM, WN, true, false, 2, BK, ST, BT, true)        \
    C3_GEMM_BF16_DE(c3_gemm_bf16_dxf_##T, WM, WN, true, true, 2, BK, ST, BT, true)          \
    C3_GEMM_BF16_DE(c3_gemm_bf16_ttf_##T, WM, WN, false, true, 2, BK, ST, BT, true)

// d256w8: 256x256 tiles, 8 waves of 128x64, 64-deep k, 2 stages (128 KiB LDS).
// Its forwards store whole tiles through LDS: timed alternately in one
// process against the direct stores (bit-identical outputs), forward
// 8192x4096x4096 249.8 -> 241.4 us, 4096x1024x4096 40.2 -> 38.2, 16384x8192x8192
// 1904 -> 1887; dX gained nothing (245.5 / 245.4, 240.4 -> 247.6), so dX,
// dW and the one-launch backward keep the direct stores.
C3_GEMM_BF16_D_KINDS_S(d256w8, 2, 4, 64, 2, 256, true)
// d128w4: 128x128 tiles, 4 waves of 64x64, 64-deep k, 2 stages (64 KiB LDS,
// two blocks per CU): four times the blocks of d256w8 for grids too small to
// fill the chip with 256x256 tiles.
// Forwards store through LDS as d256w8's do (timed against direct stores:
// 1024x1024x4096 18.2 -> 17.4 us, 4096x1024x1024 18.1 -> 17.1, 1024x4096x4096
// (4 stages) 47.6 -> 46.5; k = 8192 even).
C3_GEMM_BF16_D_KINDS_S(d128w4, 2, 2, 64, 2, 128, true)
// d128w4s4: the same tiles with 4 stages (128 KiB, one block per CU, three
// tiles in flight) for grids of one block per CU over long k.
C3_GEMM_BF16_D_KINDS_S(d128w4s4, 2, 2, 64, 4, 128, true)
// d64w4: 64x64 tiles, 4 waves of 32x32, 64-deep k, 4 stages (64 KiB): grids
// of 1024x1024 outputs, where 128x128 tiles leave three quarters of the CUs
// idle and a 2-stage pipeline exposes the memory latency at every k-tile.
C3_GEMM_BF16_D_KINDS(d64w4, 2, 2, 64, 4, 64)

// The layer backward after its pre-pass in one launch: blocks [0, nx)
// compute dX = dZ . W^T (the dx kind), [nx, nx + nw) dW = X^T . dZ (the dw
// kind), and [nx + nw, nx + nw + nf) the bias gradient's final pass over the
// pre-pass's chunk partials (64 columns per block, c3_colsum_final_f32's
// order).  A block runs one of the three bodies, so the results are those of
// the separate launches; the launch boundaries between them go.
struct Bf16BwdArgs {
    GemmArgs dx;
    GemmArgs dw;
    const float* part;  // [nchunks, dw.N] column partials (nf > 0)
    float* db;
    int64_t nchunks;
    int nx, nw;
};

// dX on one direct tile (X-suffixed parameters), dW on another with the
// same block size and LDS stages of the same size (one array, shared).
#define C3_GEMM_BF16_BWD2(NAME, WMX, WNX, STX, BTX, WMW, WNW, STW, BTW)                                     \
    extern "C" __global__ __launch_bounds__(64 * WMX * WNX) void NAME(Bf16BwdArgs p) {                     \
        static_assert(WMX * WNX == WMW * WNW, "one block size");                                             \
        __shared__ float red[8][64];                                                                          \
        const int b = blockIdx.x;                                                                             \
        if (b < p.nx)                                                                                         \
            gemm_bf16_direct_body<WMX, WNX, true, true, 0, 64, STX, BTX, BTX, true>(p.dx, b);                \
        else if (b < p.nx + p.nw)                                                                             \
            gemm_bf16_direct_body<WMW, WNW, false, false, 2, 64, STW, BTW, BTW, true>(p.dw, b - p.nx);       \
        else                                                                                                  \
            colsum_final_block<WMX * WNX>(p.part, p.db, p.nchunks, p.dw.N, b - p.nx - p.nw, red);            \
    }
#define C3_GEMM_BF16_BWD(T, WM, WN, ST, BT) C3_GEMM_BF16_BWD2(c3_gemm_bf16_bwd_##T, WM, WN, ST, BT, WM, WN, ST, BT)

C3_GEMM_BF16_BWD(d256w8, 2, 4, 2, 256)
C3_GEMM_BF16_BWD(d128w4, 2, 2, 2, 128)
C3_GEMM_BF16_BWD(d64w4, 2, 2, 4, 64)
// 64x64 and 128x128 tiles: 4 waves and 64 KiB of LDS stages each.
C3_GEMM_BF16_BWD2(c3_gemm_bf16_bwd_d64w4_d128w4, 2, 2, 4, 64, 2, 2, 2, 128)
C3_GEMM_BF16_BWD2(c3_gemm_bf16_bwd_d128w4_d64w4, 2, 2, 2, 128, 2, 2, 4, 64)



#define C3_GEMM_BF16_RQ(NAME, AK, BKC, EPI, BK, ST) \
    extern "C" __global__ __launch_bounds__(256) void NAME(GemmArgs p) { gemm_bf16_rq_body<AK, BKC, EPI, BK, ST>(split_args<AK, BKC, EPI>(p)); }
#define C3_GEMM_BF16_RQ_KINDS(T, BK, ST)                                   \
    C3_GEMM_BF16_RQ(c3_gemm_bf16_fwd_##T, true, false, 1, BK, ST)          \
    C3_GEMM_BF16_RQ(c3_gemm_bf16_dx_##T, true, true, 0, BK, ST)            \
    C3_GEMM_BF16_RQ(c3_gemm_bf16_dw_##T, false, false, 2, BK, ST)          \
    C3_GEMM_BF16_RQ(c3_gemm_bf16_dwb_##T, false, false, 0, BK, ST)         \
    C3_GEMM_BF16_RQ(c3_gemm_bf16_tt_##T, false, true, 0, BK, ST)          \
    C3_GEMM_BF16_RQ(c3_gemm_bf16_fwdt_##T, true, true, 1, BK, ST)         \
    C3_GEMM_BF16_RQ(c3_gemm_bf16_fwdf_##T, true, false, 2, BK, ST)        \
    C3_GEMM_BF16_RQ(c3_gemm_bf16_dxf_##T, true, true, 2, BK, ST)          \
    C3_GEMM_BF16_RQ(c3_gemm_bf16_ttf_##T, false, true, 2, BK, ST)

// d256rq: 64-deep k, 2 stages.
C3_GEMM_BF16_RQ_KINDS(d256rq, 64, 2)

// Split-K reduction: C[m, n] = epilogue(sum over s of ws[s * slice + m * N + n])
// with the splits added in order s = 0, 1, ... (deterministic).  Epilogue:
// + bias[n] (when non-null), act, then bf16 (round to nearest even) or fp32.
// One thread per 4 consecutive columns of a row.  With N a multiple of 4 a
// thread issues the loads of four splits before adding them (same adds, same
// order) and, when C's rows allow it, stores its 4 outputs as one vector.
struct SplitReduceArgs {
    const float* ws;
    void* C;
    const float* bias;
    int64_t M, N, ldc, slice;
    int S, act, out_bf16, _pad;
};

extern "C" __global__ __launch_bounds__(256) void c3_splitk_reduce(SplitReduceArgs a) {
    const int64_t vpr = (a.N + 3) / 4;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t m = t / vpr, n0 = 4 * (t % vpr);
    if (m >= a.M) return;
    const float* w = a.ws + m * a.N + n0;
    float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if ((a.N & 3) == 0) {
        int s = 0;
        for (; s + 4 <= a.S; s += 4) {
            f32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load((const f32x4*)(w + (int64_t)(s + u) * a.slice));
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] += v[u][e];
        }
        for (; s < a.S; ++s) {
            const f32x4 v = __builtin_nontemporal_load((const f32x4*)(w + (int64_t)s * a.slice));
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] += v[e];
        }
        if ((a.ldc & 3) == 0 && ((uintptr_t)a.C & (a.out_bf16 ? 7 : 15)) == 0) {
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                y[e] = x[e];
                if (a.bias != nullptr) y[e] = y[e] + a.bias[n0 + e];
                y[e] = act_apply(y[e], a.act);
            }
            if (a.out_bf16) {
                const unsigned lo = f32_to_bf16_rne(y[0]) | ((unsigned)f32_to_bf16_rne(y[1]) << 16);
                const unsigned hi = f32_to_bf16_rne(y[2]) | ((unsigned)f32_to_bf16_rne(y[3]) << 16);
                *(uint2*)((unsigned short*)a.C + m * a.ldc + n0) = make_uint2(lo, hi);
            } else {
                *(f32x4*)((float*)a.C + m * a.ldc + n0) = f32x4{y[0], y[1], y[2], y[3]};
            }
            return;
        }
    } else {
        for (int s = 0; s < a.S; ++s)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n0 + e < a.N) x[e] += w[(int64_t)s * a.slice + e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t n = n0 + e;
        if (n >= a.N) break;
        float y = x[e];
        if (a.bias != nullptr) y = y + a.bias[n];
        y = act_apply(y, a.act);
        if (a.out_bf16)
            ((unsigned short*)a.C)[m * a.ldc + n] = f32_to_bf16_rne(y);
        else
            ((float*)a.C)[m * a.ldc + n] = y;
    }
}

// bf16 transpose: out[c * R + r] = in[r * C + c] for in [R, C] (row-major).
// 64x64 tiles through LDS (rows padded to 72 elements): each thread loads two
// 16-byte row pieces, then gathers 8 elements of one column into a 16-byte
// store.  R and C are multiples of 8 (host-checked); edge tiles are bounded.
extern "C" __global__ __launch_bounds__(256) void c3_transpose_bf16(const unsigned short* __restrict__ in,
                                                                   unsigned short* __restrict__ out, int64_t R,
                                                                   int64_t C) {
    __shared__ __attribute__((aligned(16))) unsigned short t[64][72];
    const int tid = threadIdx.x;
    const int64_t tc = (int64_t)blockIdx.x * 64, tr = (int64_t)blockIdx.y * 64;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = tid / 8 + 32 * i, c = 8 * (tid % 8);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (tr + r < R && tc + c < C) v = __builtin_nontemporal_load((const u32x4*)(in + (tr + r) * C + tc + c));
        *(u32x4*)&t[r][c] = v;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = tid / 8 + 32 * i, r = 8 * (tid % 8);  // output row c (input column), input rows r..r+7
        if (tc + c < C && tr + r < R) {
            u32x4 w;
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = (uint32_t)t[r + 2 * j][c] | ((uint32_t)t[r + 2 * j + 1][c] << 16);
            *(u32x4*)(out + (tc + c) * R + tr + r) = w;
        }
    }
}
