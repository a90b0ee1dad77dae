// gemm_f32.hip -- fp32 GEMMs of the fused Linear(+bias)(+ReLU) layer on
// gfx950 fp32 MFMA (v_mfma_f32_32x32x2_f32), LDS double-buffered.
//
// Reference arithmetic being replaced (all fp32):
//   forward  : MatMul then FusedNode(Add -> ReLU)   src/C3/C3DialectLowering.cpp:467-610,
//                                                   src/C3/MLIRKernelGen.cpp:660-767
//   backward : ReLU mask * dY, dX = dZ.W^T, dW = X^T.dZ, db = column sum of dZ
//              src/C3/C3BackwardCapture.cpp:501-528, :618-644, :681-723
// Here the bias + activation run in the GEMM epilogue and the ReLU mask in
// the operand load, so neither the pre-activation nor dZ touches HBM.
//
// Block: NT = 64 * WAVES_M * WAVES_N threads; a wave owns a
// (BM/WAVES_M) x (BN/WAVES_N) sub-tile made of 32x32 MFMA blocks.
// One MFMA consumes one A and one B float per lane: lane l supplies
// A(row l%32, k_l) and B(k_l, col l%32) where k_l depends only on (step, l/32).
// The k order inside a 16-deep LDS tile is chosen so that each lane's eight
// k values are contiguous in LDS: step s, lane half g -> k = 8g + s.  The
// same map is used for A and B, so each output is the full sum over k.
// Output layout of a 32x32 block (16 accumulators): lane l, register v ->
// row 8*(v/4) + 4*(l/32) + v%4, column l%32.
//
// Addressing: every operand is < 4 GiB (checked on the host), so each thread
// keeps 32-bit element offsets and the k advance is a scalar pointer bump.
#include "gemm_common.h"

namespace {

constexpr int kBK = 16;   // k depth of one LDS stage
constexpr int kPad = 4;   // floats of padding per k-row of a row-contiguous tile

// LDS tile layouts.  KC (k contiguous in global): [ROWS][16 k], 64 B per row,
// the 16-byte chunk holding k 4c..4c+3 of row r stored in slot
// c ^ ((r >> 2) & 3).  A 64-byte row puts row r on bank group 4 (r & 3) +
// slot (16-byte groups, 64 banks); a ds_read_b128 serves 16 lanes = 16
// consecutive rows at a time, and (r & 3, (r >> 2) & 3) takes all 16 values
// over them, so the fragment reads are conflict-free (the key (r >> 1) & 3
// shares bit 1 with r & 3 and left a 2-way conflict); the 4-row stores stay
// conflict-free.  !KC: [16 k][ROWS + 4].
template <int ROWS, bool KC>
struct Lds {
    static constexpr int STRIDE = KC ? kBK : (ROWS + kPad);
    static constexpr int SIZE = KC ? ROWS * STRIDE : kBK * STRIDE;
    __device__ __forceinline__ static int kc_slot(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }
};

// Global -> register staging of one operand tile (ROWS x kBK logical, ROWS =
// BM for A or BN for B).  KC: k is the contiguous index in global memory.
// Each thread moves NV float4 vectors.  Out-of-range elements read as 0.
template <int ROWS, int NT, bool KC, bool MASK, bool VEC>
struct TileLoader {
    static constexpr int NVEC = ROWS * kBK / 4;
    static constexpr int NV = NVEC / NT;
    static_assert(NVEC % NT == 0, "tile must split evenly over the block");
    // KC: 4 vectors per row, vector v -> row v/4, k 4*(v%4); rows step NT/4 per i.
    // !KC: ROWS/4 vectors per k-row, vector v -> k v/(ROWS/4), row 4*(v%(ROWS/4)).
    static constexpr int RSTEP = KC ? NT / 4 : 0;
    static constexpr int KSTEP = KC ? 0 : NT / (ROWS / 4);
    static_assert(KC || NT % (ROWS / 4) == 0, "k-row split");

    f32x4 r[NV];
    uint32_t off0;   // element offset of vector 0 at k-tile 0
    uint32_t ld_;    // leading dimension (elements)
    int row0;        // tile-relative row of vector 0 (KC) / row of the vector (!KC)
    int kk0;         // tile-relative k of vector 0

    __device__ __forceinline__ void init(int tid, int64_t ld, int64_t grow0) {
        ld_ = (uint32_t)ld;
        if (KC) {
            row0 = tid >> 2;
            kk0 = 4 * (tid & 3);
            off0 = (uint32_t)((grow0 + row0) * ld + kk0);
        } else {
            kk0 = tid / (ROWS / 4);
            row0 = 4 * (tid % (ROWS / 4));
            off0 = (uint32_t)(kk0 * ld + grow0 + row0);
        }
    }

    // P/Pm already advanced to the current k-tile; rows_left = rows_total - grow0,
    // k_left = K - k0.
    __device__ __forceinline__ void load(const float* __restrict__ P, const float* __restrict__ Pm,
                                         uint32_t ld, int64_t rows_left, int64_t k_left) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int rr = KC ? row0 + i * RSTEP : row0;
            const int kk = KC ? kk0 : kk0 + i * KSTEP;
            const uint32_t off = off0 + (KC ? (uint32_t)(i * RSTEP) * ld : (uint32_t)(i * KSTEP) * ld);
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            f32x4 m = {1.f, 1.f, 1.f, 1.f};
            if (VEC) {
                if (rr < rows_left && kk < k_left) {
                    x = *(const f32x4*)(P + off);
                    if (MASK) {
                        const f32x4 y = *(const f32x4*)(Pm + off);
                        m = f32x4{relu_mask(y[0]), relu_mask(y[1]), relu_mask(y[2]), relu_mask(y[3])};
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int er = KC ? rr : rr + e;
                    const int ek = KC ? kk + e : kk;
                    if (er < rows_left && ek < k_left) {
                        const uint32_t eo = off + (uint32_t)e;
                        x[e] = P[eo];
                        if (MASK) m[e] = relu_mask(Pm[eo]);
                    }
                }
            }
            if (MASK) x = m * x;   // IEEE multiply: 0 * dY keeps dY's sign and NaN
            r[i] = x;
        }
    }

    // Write the staged (masked) values to global memory at the operand's own
    // offsets in D (advanced to the same k-tile as the load), in-range
    // elements only: the dx_mask_dz kinds write dZ this way.
    __device__ __forceinline__ void store_global(float* __restrict__ D, int64_t rows_left, int64_t k_left) const {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int rr = KC ? row0 + i * RSTEP : row0;
            const int kk = KC ? kk0 : kk0 + i * KSTEP;
            const uint32_t off = off0 + (KC ? (uint32_t)(i * RSTEP) * ld_ : (uint32_t)(i * KSTEP) * ld_);
            if (VEC) {
                if (rr < rows_left && kk < k_left) *(f32x4*)(D + off) = r[i];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int er = KC ? rr : rr + e;
                    const int ek = KC ? kk + e : kk;
                    if (er < rows_left && ek < k_left) D[off + (uint32_t)e] = r[i][e];
                }
            }
        }
    }

    __device__ __forceinline__ void store(float* __restrict__ S) const {
        constexpr int STRIDE = Lds<ROWS, KC>::STRIDE;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int rr = KC ? row0 + i * RSTEP : row0;
            const int kk = KC ? kk0 : kk0 + i * KSTEP;
            const int off = KC ? rr * STRIDE + 4 * Lds<ROWS, KC>::kc_slot(rr, kk >> 2) : kk * STRIDE + rr;
            *(f32x4*)(S + off) = r[i];
        }
    }
};

// The 4 k-values of half-step h (steps 4h..4h+3) this lane feeds to the
// 32-row MFMA block at r0.
template <int ROWS, bool KC>
__device__ __forceinline__ void read_frag(const float* __restrict__ S, int r0, int lane, int h, float (&f)[4]) {
    const int r = lane & 31, g = lane >> 5;
    constexpr int STRIDE = Lds<ROWS, KC>::STRIDE;
    if (KC) {
        const int row = r0 + r;
        const f32x4 v = *(const f32x4*)(S + row * STRIDE + 4 * Lds<ROWS, KC>::kc_slot(row, 2 * g + h));
        f[0] = v[0]; f[1] = v[1]; f[2] = v[2]; f[3] = v[3];
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) f[s] = S[(8 * g + 4 * h + s) * STRIDE + r0 + r];
    }
}

// bid: this block's index among the GEMM's blocks (see tile_coords).
// DZ: also write the masked A operand to p.dz.  Block (tm, tn) writes the
// k-tiles kt with kt % (column tiles) == tn of its rows, so every k-tile of
// every row tile is written once and the writes are spread evenly over the
// blocks; each is written from the registers that stage it into LDS.
template <int BM, int BN, int WAVES_M, int WAVES_N, bool AK, bool BKC, bool AMASK, bool BMASK,
          bool DB, bool VEC, bool DZ = false>
__device__ __forceinline__ void gemm_f32_body(const GemmArgs& p, int bid) {
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int A_SIZE = Lds<BM, AK>::SIZE, B_SIZE = Lds<BN, BKC>::SIZE;
    constexpr int STAGE = A_SIZE + B_SIZE;
    static_assert(FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tile of 32x32 blocks");

    __shared__ __attribute__((aligned(16))) float smem[2 * STAGE];
    __shared__ float db_part[DB ? NT : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn;
    tile_coords<8>(p.M, p.N, BM, BN, tm, tn, bid);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const float* __restrict__ A = (const float*)p.A;
    const float* __restrict__ Am = (const float*)p.Amask;
    const float* __restrict__ B = (const float*)p.B;
    const float* __restrict__ Bm = (const float*)p.Bmask;
    const uint32_t lda = (uint32_t)p.lda, ldb = (uint32_t)p.ldb;
    // Scalar advance of the operand base per k-tile.
    const int64_t a_kstep = AK ? kBK : (int64_t)kBK * p.lda;
    const int64_t b_kstep = BKC ? kBK : (int64_t)kBK * p.ldb;

    TileLoader<BM, NT, AK, AMASK, VEC> la;
    TileLoader<BN, NT, BKC, BMASK, VEC> lb;
    la.init(tid, p.lda, m0);
    lb.init(tid, p.ldb, n0);
    const int64_t a_rows = p.M - m0, b_rows = p.N - n0;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // db: the block on the first row-tile sums the masked B operand over all k.
    const bool do_db = DB && p.db != nullptr && tm == 0;
    float dbacc = 0.0f;

    const int nk = (int)((p.K + kBK - 1) / kBK);
    float* __restrict__ Dz = (float*)p.dz;
    const int nbn = (int)((p.N + BN - 1) / BN);
    la.load(A, Am, lda, a_rows, p.K);
    lb.load(B, Bm, ldb, b_rows, p.K);
    if (DZ && tn == 0) la.store_global(Dz, a_rows, p.K);
    la.store(smem);
    lb.store(smem + A_SIZE);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const float* As = smem + cur * STAGE;
        const float* Bs = As + A_SIZE;
        const bool more = kt + 1 < nk;
        if (more) {
            const int64_t k0 = (int64_t)(kt + 1) * kBK;
            const int64_t ao = (int64_t)(kt + 1) * a_kstep, bo = (int64_t)(kt + 1) * b_kstep;
            la.load(A + ao, AMASK ? Am + ao : Am, lda, a_rows, p.K - k0);
            lb.load(B + bo, BMASK ? Bm + bo : Bm, ldb, b_rows, p.K - k0);
        }

#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // Two half-steps of 4 k-values keep fewer fragment registers live.
            float af[FM][4], bf[FN][4];
#pragma unroll
            for (int i = 0; i < FM; ++i) read_frag<BM, AK>(As, wm * TM + 32 * i, lane, h, af[i]);
#pragma unroll
            for (int j = 0; j < FN; ++j) read_frag<BN, BKC>(Bs, wn * TN + 32 * j, lane, h, bf[j]);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
        }

        if (DB && do_db) {
            // B tile is stored [k][n] (!BKC): thread -> column tid % BN.
            static_assert(!DB || !BKC, "db side output needs the [k][n] B tile");
            static_assert(!DB || NT % BN == 0, "threads per column");
            constexpr int RPT = NT / BN;
            const int c = tid % BN, rs = tid / BN;
#pragma unroll
            for (int k = rs; k < kBK; k += RPT) dbacc += Bs[k * Lds<BN, false>::STRIDE + c];
        }

        if (more) {
            float* Ns = smem + (cur ^ 1) * STAGE;
            if (DZ && (kt + 1) % nbn == tn)
                la.store_global(Dz + (int64_t)(kt + 1) * a_kstep, a_rows, p.K - (int64_t)(kt + 1) * kBK);
            la.store(Ns);
            lb.store(Ns + A_SIZE);
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

    // Epilogue: bias add then activation, straight from the accumulators.
    float* __restrict__ C = (float*)p.C;
    const int r = lane & 31, g = lane >> 5;
    auto store_all = [&](auto actf) {
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
                        C[m * p.ldc + n] = actf(x);
                    }
                }
            }
        }
    };
    if constexpr (BM * BN <= 64 * 64) {
        // Small tiles run on grids of a few blocks, where each launch pays for
        // fetching its code: the activation is chosen once per block so the
        // stores carry only that activation's instructions (the per-element
        // form puts the sigmoid and tanh code at each of the 16 stores).
        with_act(p.act, [&](auto at) {
            constexpr int ACT = decltype(at)::value;
            store_all([](float x) { return act_c<ACT>(x); });
        });
    } else {
        // Large tiles: the per-element form keeps the VGPR count (and so the
        // occupancy) the MFMA loop needs.
        store_all([&](float x) { return act_apply(x, p.act); });
    }
}

}  // namespace

namespace {
// Split-K: block row blockIdx.y multiplies k in [y * split_k, y * split_k +
// split_k) (the masks follow their operands) and writes the raw partial
// product to C + y * c_split; the host passes no bias, activation or db, and
// c3_splitk_reduce adds the partials and applies the epilogue.
template <bool AK, bool BKC>
__device__ __forceinline__ GemmArgs split_args_f32(const GemmArgs& p) {
    if (p.split_k == 0) return p;
    GemmArgs q = p;
    const int64_t k0 = (int64_t)blockIdx.y * p.split_k;
    const int64_t ao = AK ? k0 : k0 * p.lda, bo = BKC ? k0 : k0 * p.ldb;
    q.A = (const float*)p.A + ao;
    if (p.Amask) q.Amask = (const float*)p.Amask + ao;
    q.B = (const float*)p.B + bo;
    if (p.Bmask) q.Bmask = (const float*)p.Bmask + bo;
    q.K = min(p.split_k, p.K - k0);
    q.C = (float*)p.C + (int64_t)blockIdx.y * p.c_split;
    return q;
}
}  // namespace

// One extern "C" symbol per (layout, fusion, tile, vector) case.
// Tile suffix _tBMxBN_wWMxWN; _v: vectorised operand loads (contiguous extent
// % 4 == 0 and 16-byte aligned bases), _s: scalar loads.
#define C3_GEMM_F32_ONE_DZ(NAME, BM, BN, WM, WN, OCC, AK, BKC, AMASK, BMASK, DB, DZ)                              \
    extern "C" __global__ __launch_bounds__(64 * WM * WN, OCC) void NAME##_v(GemmArgs p) {                         \
        gemm_f32_body<BM, BN, WM, WN, AK, BKC, AMASK, BMASK, DB, true, DZ>(split_args_f32<AK, BKC>(p), blockIdx.x);  \
    }                                                                                                             \
    extern "C" __global__ __launch_bounds__(64 * WM * WN, OCC) void NAME##_s(GemmArgs p) {                         \
        gemm_f32_body<BM, BN, WM, WN, AK, BKC, AMASK, BMASK, DB, false, DZ>(split_args_f32<AK, BKC>(p), blockIdx.x); \
    }
#define C3_GEMM_F32_ONE(NAME, BM, BN, WM, WN, OCC, AK, BKC, AMASK, BMASK, DB) \
    C3_GEMM_F32_ONE_DZ(NAME, BM, BN, WM, WN, OCC, AK, BKC, AMASK, BMASK, DB, false)

// Kinds: fwd (A=X k-contig, B=W [K,N]); dx/dx_mask (A=dY[, masked by Y], B=W as [N][K]);
// dx_mask_dz (dx_mask that also writes dZ = the masked dY); dw/dw_mask (A=X^T,
// B=dY[, masked]; db side output); tt (A^T . B^T).
#define C3_GEMM_F32_KINDS(T, BM, BN, WM, WN, OCC)                                                    \
    C3_GEMM_F32_ONE(c3_gemm_f32_fwd_##T, BM, BN, WM, WN, OCC, true, false, false, false, false)      \
    C3_GEMM_F32_ONE(c3_gemm_f32_dx_##T, BM, BN, WM, WN, OCC, true, true, false, false, false)        \
    C3_GEMM_F32_ONE(c3_gemm_f32_dx_mask_##T, BM, BN, WM, WN, OCC, true, true, true, false, false)    \
    C3_GEMM_F32_ONE_DZ(c3_gemm_f32_dx_mask_dz_##T, BM, BN, WM, WN, OCC, true, true, true, false, false, true) \
    C3_GEMM_F32_ONE(c3_gemm_f32_dw_##T, BM, BN, WM, WN, OCC, false, false, false, false, true)       \
    C3_GEMM_F32_ONE(c3_gemm_f32_dw_mask_##T, BM, BN, WM, WN, OCC, false, false, false, true, true)   \
    C3_GEMM_F32_ONE(c3_gemm_f32_tt_##T, BM, BN, WM, WN, OCC, false, true, false, false, false)

C3_GEMM_F32_KINDS(t64x64, 64, 64, 2, 2, 2)
C3_GEMM_F32_KINDS(t128x128, 128, 128, 2, 2, 2)
C3_GEMM_F32_KINDS(t256x128, 256, 128, 4, 2, 1)
C3_GEMM_F32_KINDS(t128x256, 128, 256, 2, 4, 1)

// The whole layer backward of a small layer in one launch: blocks
// [0, nx) compute dX = dZ . W^T (dx kind), blocks [nx, nx + nw) dW = X^T . dZ
// with db (dw kind), each with its own tile walk; a block runs one of the
// two bodies, so results are those of the two separate launches.  For grids
// of a few 64x64 tiles, where each launch costs more than its k-loop.
struct BwdPairArgs {
    GemmArgs dx;
    GemmArgs dw;
    int nx;
    int _pad;
};

#define C3_GEMM_F32_BWD_PAIR(NAME, BM, BN, WM, WN, OCC, MASK, VEC)                                              \
    extern "C" __global__ __launch_bounds__(64 * WM * WN, OCC) void NAME(BwdPairArgs p) {                      \
        const int b = blockIdx.x;                                                                              \
        if (b < p.nx)                                                                                          \
            gemm_f32_body<BM, BN, WM, WN, true, true, MASK, false, false, VEC>(p.dx, b);                      \
        else                                                                                                   \
            gemm_f32_body<BM, BN, WM, WN, false, false, false, MASK, true, VEC>(p.dw, b - p.nx);              \
    }

C3_GEMM_F32_BWD_PAIR(c3_gemm_f32_bwd_t64x64_v, 64, 64, 2, 2, 2, false, true)
C3_GEMM_F32_BWD_PAIR(c3_gemm_f32_bwd_t64x64_s, 64, 64, 2, 2, 2, false, false)
C3_GEMM_F32_BWD_PAIR(c3_gemm_f32_bwd_mask_t64x64_v, 64, 64, 2, 2, 2, true, true)
C3_GEMM_F32_BWD_PAIR(c3_gemm_f32_bwd_mask_t64x64_s, 64, 64, 2, 2, 2, true, false)
