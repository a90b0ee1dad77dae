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

// Epilogue shared by the register-staged and direct kernels: the db column
// sums (block on the first row-tile, dbacc = this thread's partial of column
// tid % BN), then bias add and activation straight from the accumulators.
// Accumulator layout of a 32x32 block: lane l, register v -> row
// 8*(v/4) + 4*(l/32) + v%4, column l%32.
template <int BM, int BN, int WAVES_M, int WAVES_N, bool DB>
__device__ __forceinline__ void f32_tile_epilogue(const GemmArgs& p, f32x16 (&acc)[BM / WAVES_M / 32][BN / WAVES_N / 32],
                                                  int64_t m0, int64_t n0, int wm, int wn, int tid, int lane,
                                                  bool do_db, float dbacc, float* db_part) {
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;
    constexpr int FM = TM / 32, FN = TN / 32;
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

// bid: this block's index among the GEMM's blocks (see tile_coords).
// DZ: also write the masked A operand to p.dz.  Block (tm, tn) writes the
// k-tiles kt with kt % (column tiles) == tn of its rows, so every k-tile of
// every row tile is written once and the writes are spread evenly over the
// blocks; each is written from the registers that stage it into LDS.
// KALL > 0: every k-tile at once (the host launches these kernels only when
// K <= 16 * KALL): all tiles' loads are issued together into registers, each
// tile stored to its own LDS stage and one barrier taken, so the k range
// costs one memory round trip instead of one per k-tile; the multiplies, the
// db sums and the dZ writes are those of the loop, in the same order.
template <int BM, int BN, int WAVES_M, int WAVES_N, bool AK, bool BKC, bool AMASK, bool BMASK,
          bool DB, bool VEC, bool DZ = false, int KALL = 0>
__device__ __forceinline__ void gemm_f32_body(const GemmArgs& p, int bid) {
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int A_SIZE = Lds<BM, AK>::SIZE, B_SIZE = Lds<BN, BKC>::SIZE;
    constexpr int STAGE = A_SIZE + B_SIZE;
    static_assert(FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tile of 32x32 blocks");

    __shared__ __attribute__((aligned(16))) float smem[(KALL > 0 ? KALL : 2) * STAGE];
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

    // One k-tile's multiplies from its LDS stage, and the db sums over it.
    auto multiply = [&](const float* As, const float* Bs) {
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
    };

    if constexpr (KALL > 0) {
        TileLoader<BM, NT, AK, AMASK, VEC> las[KALL];
        TileLoader<BN, NT, BKC, BMASK, VEC> lbs[KALL];
#pragma unroll
        for (int t = 0; t < KALL; ++t) {
            las[t] = la;
            lbs[t] = lb;
            if (t < nk) {
                const int64_t ao = (int64_t)t * a_kstep, bo = (int64_t)t * b_kstep;
                las[t].load(A + ao, AMASK ? Am + ao : Am, lda, a_rows, p.K - (int64_t)t * kBK);
                lbs[t].load(B + bo, BMASK ? Bm + bo : Bm, ldb, b_rows, p.K - (int64_t)t * kBK);
            }
        }
#pragma unroll
        for (int t = 0; t < KALL; ++t) {
            if (t < nk) {
                if (DZ && t % nbn == tn)
                    las[t].store_global(Dz + (int64_t)t * a_kstep, a_rows, p.K - (int64_t)t * kBK);
                las[t].store(smem + t * STAGE);
                lbs[t].store(smem + t * STAGE + A_SIZE);
            }
        }
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) multiply(smem + kt * STAGE, smem + kt * STAGE + A_SIZE);
        f32_tile_epilogue<BM, BN, WAVES_M, WAVES_N, DB>(p, acc, m0, n0, wm, wn, tid, lane, do_db, dbacc, db_part);
        return;
    }

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

        multiply(As, Bs);

        if (more) {
            float* Ns = smem + (cur ^ 1) * STAGE;
            if (DZ && (kt + 1) % nbn == tn)
                la.store_global(Dz + (int64_t)(kt + 1) * a_kstep, a_rows, p.K - (int64_t)(kt + 1) * kBK);
            la.store(Ns);
            lb.store(Ns + A_SIZE);
        }
        __syncthreads();
    }

    f32_tile_epilogue<BM, BN, WAVES_M, WAVES_N, DB>(p, acc, m0, n0, wm, wn, tid, lane, do_db, dbacc, db_part);
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
#define C3_GEMM_F32_ONE_DZK(NAME, BM, BN, WM, WN, OCC, AK, BKC, AMASK, BMASK, DB, DZ, KA)                                 \
    extern "C" __global__ __launch_bounds__(64 * WM * WN, OCC) void NAME##_v(GemmArgs p) {                               \
        gemm_f32_body<BM, BN, WM, WN, AK, BKC, AMASK, BMASK, DB, true, DZ, KA>(split_args_f32<AK, BKC>(p), blockIdx.x);  \
    }                                                                                                                   \
    extern "C" __global__ __launch_bounds__(64 * WM * WN, OCC) void NAME##_s(GemmArgs p) {                               \
        gemm_f32_body<BM, BN, WM, WN, AK, BKC, AMASK, BMASK, DB, false, DZ, KA>(split_args_f32<AK, BKC>(p), blockIdx.x); \
    }
#define C3_GEMM_F32_ONE_DZ(NAME, BM, BN, WM, WN, OCC, AK, BKC, AMASK, BMASK, DB, DZ) \
    C3_GEMM_F32_ONE_DZK(NAME, BM, BN, WM, WN, OCC, AK, BKC, AMASK, BMASK, DB, DZ, 0)
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
// t64x64k: the 64x64 kinds with every k-tile loaded at once, for K <= 128
// (eight 16-deep k-tiles, eight LDS stages), vector-aligned operands only
// (the scalar-load form measured slower: its many predicated loads and
// larger code cost more than the round trips they save).
#define C3_GEMM_F32_ONE_VK(NAME, BM, BN, WM, WN, OCC, AK, BKC, AMASK, BMASK, DB, DZ, KA)                                 \
    extern "C" __global__ __launch_bounds__(64 * WM * WN, OCC) void NAME##_v(GemmArgs p) {                               \
        gemm_f32_body<BM, BN, WM, WN, AK, BKC, AMASK, BMASK, DB, true, DZ, KA>(split_args_f32<AK, BKC>(p), blockIdx.x);  \
    }
#define C3_GEMM_F32_KINDS_KALL(T, BM, BN, WM, WN, OCC, KA)                                                         \
    C3_GEMM_F32_ONE_VK(c3_gemm_f32_fwd_##T, BM, BN, WM, WN, OCC, true, false, false, false, false, false, KA)      \
    C3_GEMM_F32_ONE_VK(c3_gemm_f32_dx_##T, BM, BN, WM, WN, OCC, true, true, false, false, false, false, KA)        \
    C3_GEMM_F32_ONE_VK(c3_gemm_f32_dx_mask_##T, BM, BN, WM, WN, OCC, true, true, true, false, false, false, KA)    \
    C3_GEMM_F32_ONE_VK(c3_gemm_f32_dx_mask_dz_##T, BM, BN, WM, WN, OCC, true, true, true, false, false, true, KA)  \
    C3_GEMM_F32_ONE_VK(c3_gemm_f32_dw_##T, BM, BN, WM, WN, OCC, false, false, false, false, true, false, KA)       \
    C3_GEMM_F32_ONE_VK(c3_gemm_f32_dw_mask_##T, BM, BN, WM, WN, OCC, false, false, false, true, true, false, KA)   \
    C3_GEMM_F32_ONE_VK(c3_gemm_f32_tt_##T, BM, BN, WM, WN, OCC, false, true, false, false, false, false, KA)
C3_GEMM_F32_KINDS_KALL(t64x64k, 64, 64, 2, 2, 2, 8)
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

#define C3_GEMM_F32_BWD_PAIR_K(NAME, BM, BN, WM, WN, OCC, MASK, VEC, KA)                                        \
    extern "C" __global__ __launch_bounds__(64 * WM * WN, OCC) void NAME(BwdPairArgs p) {                      \
        const int b = blockIdx.x;                                                                              \
        if (b < p.nx)                                                                                          \
            gemm_f32_body<BM, BN, WM, WN, true, true, MASK, false, false, VEC, false, KA>(p.dx, b);           \
        else                                                                                                   \
            gemm_f32_body<BM, BN, WM, WN, false, false, false, MASK, true, VEC, false, KA>(p.dw, b - p.nx);   \
    }
#define C3_GEMM_F32_BWD_PAIR(NAME, BM, BN, WM, WN, OCC, MASK, VEC) C3_GEMM_F32_BWD_PAIR_K(NAME, BM, BN, WM, WN, OCC, MASK, VEC, 0)

C3_GEMM_F32_BWD_PAIR(c3_gemm_f32_bwd_t64x64_v, 64, 64, 2, 2, 2, false, true)
C3_GEMM_F32_BWD_PAIR(c3_gemm_f32_bwd_t64x64_s, 64, 64, 2, 2, 2, false, false)
C3_GEMM_F32_BWD_PAIR(c3_gemm_f32_bwd_mask_t64x64_v, 64, 64, 2, 2, 2, true, true)
C3_GEMM_F32_BWD_PAIR(c3_gemm_f32_bwd_mask_t64x64_s, 64, 64, 2, 2, 2, true, false)
// Both GEMMs with k <= 128, vector-aligned: every k-tile at once.
C3_GEMM_F32_BWD_PAIR_K(c3_gemm_f32_bwd_t64x64k_v, 64, 64, 2, 2, 2, false, true, 8)
C3_GEMM_F32_BWD_PAIR_K(c3_gemm_f32_bwd_mask_t64x64k_v, 64, 64, 2, 2, 2, true, true, 8)

// ===========================================================================
// Direct-to-LDS fp32 kernels (tiles t256x128d, t128x256d): the operand tiles go from global
// memory straight into LDS with global_load_lds_dwordx4 (lane l's 16 bytes
// land at M0 + 16 l of the instruction's 1 KiB), three LDS stages, two tiles
// in flight ahead of the one multiplied.  The register-staged kernels above
// prefetch one tile ahead through VGPRs, and the compiler waits for every
// outstanding load before the LDS stores (their loads are predicated), so the
// memory latency of each k-tile is exposed at its end; timed on MI355X at
// 8192x4096x4096, the same kernels with the next tile's loads taken out run
// 11% (forward), 15% (dX) and 8% (dW) faster, which is the room this path
// is for.  The MFMA sequence, fragment mapping and k order are those of the
// register kernels, so the outputs are bit-identical to theirs.
//
// LDS layouts (one 16-deep k-tile of ROWS rows):
//   KC: [ROWS][16], chunk c (k 4c..4c+3) of row r in slot c ^ ((r >> 2) & 3),
//       the register kernels' layout; DMA instruction q fills rows
//       16q..16q+15 and lane l fetches the global chunk that its slot holds.
//   RC: [16 k][ROWS] with 128 bytes inserted before k-row 8, so k-rows kr and
//       kr + 8 (read by the two lane halves of one fragment read) sit 32
//       banks apart; the register kernels get that from a 4-float pad per
//       k-row, which a DMA instruction (1 KiB contiguous) cannot leave.
// Requires K % 16 == 0, K >= 16, contiguous extents % 4 == 0 and 16-byte
// aligned operands (host-checked); rows or columns past M or N are loaded
// from a clamped address and never stored.
// ===========================================================================
namespace {

template <int ROWS, bool KC, int NW>
struct F32DirectTile {
    static constexpr int CPR = KC ? 4 : ROWS / 4;      // 16-byte chunks per LDS row (KC) / k-row (RC)
    static constexpr int NQ = ROWS * kBK * 4 / 1024;   // 1 KiB DMA instructions per tile
    static constexpr int NI = NQ / NW;                 // per wave
    static constexpr int GAP = KC ? 0 : 32;            // floats before k-row 8 (RC)
    static constexpr int FLOATS = ROWS * kBK + GAP;    // LDS floats of one tile
    static_assert(NQ % NW == 0, "tile must split into whole instructions per wave");
    static_assert(KC || (CPR <= 64 && 64 % CPR == 0), "RC: whole k-rows per instruction");
    uint32_t goff[NI];

    // LDS byte offset of instruction q inside the tile.
    __device__ __forceinline__ static constexpr uint32_t qoff(int q) {
        return (uint32_t)(q * 1024 + ((!KC && q * (64 / CPR) >= 8) ? 4 * GAP : 0));
    }

    __device__ __forceinline__ void init(int wave, int lane, int64_t ld, int64_t grow0, int64_t rows_total) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int q = wave * NI + i;
            if (KC) {
                const int r = 16 * q + lane / 4;
                const int c = (lane & 3) ^ ((r >> 2) & 3);
                int64_t gr = grow0 + r;
                if (gr > rows_total - 1) gr = rows_total - 1;
                goff[i] = (uint32_t)(gr * ld + 4 * c);
            } else {
                const int kr = q * (64 / CPR) + lane / CPR;
                int64_t gc = grow0 + 4 * (lane % CPR);
                if (gc > rows_total - 4) gc = rows_total - 4;
                goff[i] = (uint32_t)(kr * ld + gc);
            }
        }
    }

    // P advanced to the k-tile; s_lds = LDS byte address of this operand's tile.
    // Issued through inline asm (M0 = the instruction's LDS destination), so
    // the compiler does not count them; the kernel waits with s_waitcnt vmcnt.
    __device__ __forceinline__ void issue(const float* P, uint32_t s_lds, int wave) const {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t lds = s_lds + qoff(wave * NI + i);
            const float* src = P + goff[i];
            asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                         :
                         : "s"(lds), "v"(src)
                         : "memory", "m0");
        }
    }

    // The 4 k-values of half-step h this lane feeds to the 32-row MFMA block
    // at r0 (k = 8 (lane / 32) + 4h + s, as in read_frag).
    __device__ __forceinline__ static void frag(const float* __restrict__ S, int r0, int lane, int h, float (&f)[4]) {
        const int r = lane & 31, g = lane >> 5;
        if (KC) {
            read_frag<ROWS, true>(S, r0, lane, h, f);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) f[s] = S[(8 * g + 4 * h + s) * ROWS + GAP * g + r0 + r];
        }
    }

    // Element (k, row) of an RC tile (the db column sums).
    __device__ __forceinline__ static float at(const float* __restrict__ S, int k, int row) {
        return S[k * ROWS + (k >= 8 ? GAP : 0) + row];
    }
};

// s_waitcnt vmcnt(n) alone (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void f32_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait until at most min(after, J) tiles' DMA instructions (NIW per tile)
// are outstanding.
template <int NIW, int J>
__device__ __forceinline__ void f32_wait_tiles_upto(int after) {
    if constexpr (J == 0) {
        f32_wait_vmcnt<0>();
    } else {
        if (after >= J) f32_wait_vmcnt<J * NIW>();
        else f32_wait_tiles_upto<NIW, J - 1>(after);
    }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, bool AK, bool BKC, bool DB, bool EARLY = false, int STAGES = 3>
__device__ __forceinline__ void gemm_f32_direct_body(const GemmArgs& p) {
    constexpr int NT = 64 * WAVES_M * WAVES_N, NW = WAVES_M * WAVES_N;
    constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int PF = STAGES - 1;
    using TA = F32DirectTile<BM, AK, NW>;
    using TB = F32DirectTile<BN, BKC, NW>;
    constexpr int STAGE = TA::FLOATS + TB::FLOATS;
    constexpr int NIW = TA::NI + TB::NI;
    static_assert(PF * NIW < 64, "outstanding DMA instructions exceed vmcnt");
    static_assert((STAGE * 4) % 16 == 0, "stages stay 16-byte aligned");

    __shared__ __attribute__((aligned(1024))) float smem[STAGES * STAGE];
    __shared__ float db_part[DB ? NT : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn;
    tile_coords<8>(p.M, p.N, BM, BN, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const float* A = (const float*)p.A;
    const float* B = (const float*)p.B;
    TA la;
    TB lb;
    la.init(wave, lane, p.lda, m0, p.M);
    lb.init(wave, lane, p.ldb, n0, p.N);
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

    const int nk = (int)(p.K / kBK);
    const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)smem);
    auto issue_tile = [&](int t, int stage) {
        const uint32_t sl = smem_lds + (uint32_t)(stage * STAGE * 4);
        la.issue(A + (int64_t)t * a_kstep, sl, wave);
        lb.issue(B + (int64_t)t * b_kstep, sl + (uint32_t)(TA::FLOATS * 4), wave);
    };
#pragma unroll
    for (int t = 0; t < PF; ++t) {
        if (t < nk) issue_tile(t, t);
    }

    for (int kt = 0; kt < nk; ++kt) {
        // Tile kt has landed when at most the DMA of the tiles issued after
        // it (min(nk - 1 - kt, PF - 1) of them) is outstanding; the barrier
        // then makes every wave's part visible and ends every read of the
        // stage refilled below (tile kt - 1's).
        f32_wait_tiles_upto<NIW, PF - 1>(min(nk - 1 - kt, PF - 1));
        __syncthreads();
        const float* As = smem + (kt % STAGES) * STAGE;
        const float* Bs = As + TA::FLOATS;
        float af0[FM][4], bf0[FN][4];
        if (EARLY) {
#pragma unroll
            for (int i = 0; i < FM; ++i) TA::frag(As, wm * TM + 32 * i, lane, 0, af0[i]);
#pragma unroll
            for (int j = 0; j < FN; ++j) TB::frag(Bs, wn * TN + 32 * j, lane, 0, bf0[j]);
        }
        if (kt + PF < nk) issue_tile(kt + PF, (kt + PF) % STAGES);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float af[FM][4], bf[FN][4];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                if (EARLY && h == 0) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) af[i][s] = af0[i][s];
                } else {
                    TA::frag(As, wm * TM + 32 * i, lane, h, af[i]);
                }
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if (EARLY && h == 0) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) bf[j][s] = bf0[j][s];
                } else {
                    TB::frag(Bs, wn * TN + 32 * j, lane, h, bf[j]);
                }
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
        }
        if (DB && do_db) {
            static_assert(!DB || !BKC, "db side output needs the [k][n] B tile");
            static_assert(!DB || NT % BN == 0, "threads per column");
            constexpr int RPT = NT / BN;
            const int c = tid % BN, rs = tid / BN;
#pragma unroll
            for (int k = rs; k < kBK; k += RPT) dbacc += TB::at(Bs, k, c);
        }
    }
    f32_tile_epilogue<BM, BN, WAVES_M, WAVES_N, DB>(p, acc, m0, n0, wm, wn, tid, lane, do_db, dbacc, db_part);
}

}  // namespace

#define C3_GEMM_F32_D(NAME, BM, BN, WM, WN, AK, BKC, DB, E)                                \
    extern "C" __global__ __launch_bounds__(64 * WM * WN, 1) void NAME(GemmArgs p) {       \
        gemm_f32_direct_body<BM, BN, WM, WN, AK, BKC, DB, E>(p);                            \
    }
// With ST LDS stages and split-K (block row y takes its k range, as the
// register kernels do).
#define C3_GEMM_F32_DS(NAME, BM, BN, WM, WN, AK, BKC, DB, E, ST)                              \
    extern "C" __global__ __launch_bounds__(64 * WM * WN) void NAME(GemmArgs p) {              \
        gemm_f32_direct_body<BM, BN, WM, WN, AK, BKC, DB, E, ST>(split_args_f32<AK, BKC>(p));    \
    }
// fwd: X (KC) . W (RC); dx: dZ (KC) . W^T (KC); dw: X^T (RC) . dZ (RC), db
// when p.db is set.  The dX kinds issue each tile's first fragment reads
// before the next tile's DMA (EARLY); measured on MI355X at 8192x4096x4096
// that order gains 6% on dX and loses 1% on the forward and 8% on dW.
#define C3_GEMM_F32_D_KINDS(T, BM, BN, WM, WN)                                       \
    C3_GEMM_F32_D(c3_gemm_f32_fwd_##T, BM, BN, WM, WN, true, false, false, false)   \
    C3_GEMM_F32_D(c3_gemm_f32_dx_##T, BM, BN, WM, WN, true, true, false, true)      \
    C3_GEMM_F32_D(c3_gemm_f32_dw_##T, BM, BN, WM, WN, false, false, true, false)

C3_GEMM_F32_D_KINDS(t256x128d, 256, 128, 4, 2)
C3_GEMM_F32_D_KINDS(t128x256d, 128, 256, 2, 4)
// 256x256: 8 waves of 128x64, one block per CU (98 KiB of LDS), half the
// operand bytes per flop of the tiles above; taken for dX and dW on grids of
// at least 256 such tiles (measured at 8192x4096x4096, alternating in one
// process: dX 141.0 against 138.7 TFLOP/s, dW 139.6 against 138.7; the
// forward is faster on 256x128, 139.2 against 137.9).
C3_GEMM_F32_D(c3_gemm_f32_dx_t256x256d, 256, 256, 2, 4, true, true, false, true)
C3_GEMM_F32_D(c3_gemm_f32_dw_t256x256d, 256, 256, 2, 4, false, false, true, false)
// 64x64: 4 waves of 32x32 and 6 LDS stages (five tiles in flight, 50 KiB)
// for the small grids of the 64x64 register tile, whose k loop is a chain
// of dependent memory round trips.
C3_GEMM_F32_DS(c3_gemm_f32_fwd_t64x64d, 64, 64, 2, 2, true, false, false, false, 6)
C3_GEMM_F32_DS(c3_gemm_f32_dx_t64x64d, 64, 64, 2, 2, true, true, false, true, 6)
C3_GEMM_F32_DS(c3_gemm_f32_dw_t64x64d, 64, 64, 2, 2, false, false, true, false, 6)
