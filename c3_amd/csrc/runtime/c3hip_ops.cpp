// c3hip_ops.cpp -- argument checking and kernel selection behind the compute
// entry points of include/c3hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <string>

#include "c3hip.h"
#include "c3hip_internal.h"

namespace c3hip {
namespace {

constexpr int64_t kMaxElems32 = (int64_t)1 << 32;  // GEMM operands use 32-bit element offsets

const char* ew_name(int op) {
    switch (op) {
        case C3HIP_EW_ADD: return "add";
        case C3HIP_EW_SUB: return "sub";
        case C3HIP_EW_MUL: return "mul";
        case C3HIP_EW_DIV: return "div";
        case C3HIP_EW_RELU: return "relu";
        case C3HIP_EW_RELU_BWD: return "relu_bwd";
        case C3HIP_EW_NEG: return "neg";
        case C3HIP_EW_SCALE: return "scale";
        case C3HIP_EW_SIGMOID: return "sigmoid";
        case C3HIP_EW_TANH: return "tanh";
        case C3HIP_EW_EXP: return "exp";
        case C3HIP_EW_LOG: return "log";
        case C3HIP_EW_SIGMOID_BWD: return "sigmoid_bwd";
        case C3HIP_EW_TANH_BWD: return "tanh_bwd";
        case C3HIP_EW_EXP_BWD: return "exp_bwd";
        default: return nullptr;
    }
}

bool ew_is_binary(int op) {
    return op == C3HIP_EW_ADD || op == C3HIP_EW_SUB || op == C3HIP_EW_MUL || op == C3HIP_EW_DIV ||
           op == C3HIP_EW_RELU_BWD || op == C3HIP_EW_SIGMOID_BWD || op == C3HIP_EW_TANH_BWD ||
           op == C3HIP_EW_EXP_BWD;
}

// ---- GEMM planning -------------------------------------------------------

enum class Kind { Fwd, FwdT, Dx, DxMask, DxMaskDz, Dw, DwMask, DwB, TT };

const char* kind_name(Kind k) {
    switch (k) {
        case Kind::Fwd: return "fwd";
        case Kind::FwdT: return "fwdt";
        case Kind::Dx: return "dx";
        case Kind::DxMask: return "dx_mask";
        case Kind::DxMaskDz: return "dx_mask_dz";
        case Kind::Dw: return "dw";
        case Kind::DwMask: return "dw_mask";
        case Kind::DwB: return "dwb";
        case Kind::TT: return "tt";
    }
    return "?";
}

struct Tile {
    const char* name;
    int bm, bn, threads;
    int bk;             // k depth of one tile (direct-to-LDS kernels); 0 = any K
    bool ktail = false;  // direct kernel takes a partial last k-tile (else K must be a multiple of bk)
};

// Threads per block of the vector elementwise and backward-chain kernels
// (elementwise.hip kVecThreads): one float4 per thread.
constexpr int64_t kEwVecThreads = 64;

// The last four are direct-to-LDS tiles (gemm_f32.hip, names ending in d):
// the twins of the register-staged 256x128 and 128x256 tiles (same blocks and
// bits), a 256x256 tile for dX and dW and a 64x64 tile with 6 LDS stages,
// taken for unmasked GEMMs with K % 16 == 0 (f32_direct).  Every fp32 tile multiplies each output's k range
// in the same order, so all of them give the same bits.
const Tile kF32Tiles[] = {{"t64x64", 64, 64, 256},        {"t128x128", 128, 128, 256}, {"t256x128", 256, 128, 512},
                          {"t128x256", 128, 256, 512},    {"t256x128d", 256, 128, 512, 16},
                          {"t128x256d", 128, 256, 512, 16}, {"t256x256d", 256, 256, 512, 16},
                          {"t64x64d", 64, 64, 256, 16}};
const Tile kBf16Tiles[] = {{"t64x64", 64, 64, 256},
                           {"t128x128", 128, 128, 256},
                           {"t256x128", 256, 128, 256},
                           {"t256x256", 256, 256, 256}};

const Tile* find_tile(const Tile* tiles, size_t n, const char* name) {
    for (size_t i = 0; i < n; ++i)
        if (std::strcmp(tiles[i].name, name) == 0) return &tiles[i];
    return nullptr;
}

// Tile forced for the calling thread (c3hip_set_gemm_tile); empty = none.
thread_local std::string t_tile_f32, t_tile_bf16;

// fp32 tile per GEMM kind and size (c3hip_set_gemm_tile, then C3_HIP_GEMM_TILE, override it).  Measured on MI355X at 8192x4096x4096
// (tiles timed alternately in one process, TFLOP/s for 128x128 / 256x128 /
// 128x256 / 256x256, the last measured and not built): forward 127-129 / 132-133 / 133 / 133; dX with the ReLU
// mask 118-120 / 115-116 / 125-126 / 109; dW with mask and db 111-113 / 121-122
// / 115-116 / 105.  dX stages two A operands (dY and Y for the mask), so the
// tile that is wide in N loads the fewest of them per flop; dW reads A k-major
// down k = M.  Small grids use 64x64 so every CU gets a block.
bool f32_forced() { return !t_tile_f32.empty() || std::getenv("C3_HIP_GEMM_TILE") != nullptr; }

const Tile* choose_f32_tile(Kind kind, int64_t M, int64_t N) {
    const size_t nt = sizeof(kF32Tiles) / sizeof(kF32Tiles[0]);
    const char* forced = !t_tile_f32.empty() ? t_tile_f32.c_str() : std::getenv("C3_HIP_GEMM_TILE");
    if (forced) {
        if (const Tile* t = find_tile(kF32Tiles, nt, forced)) return t;
    }
    const bool dw = kind == Kind::Dw || kind == Kind::DwMask;
    const bool dx = kind == Kind::Dx || kind == Kind::DxMask || kind == Kind::DxMaskDz;
    const int64_t blocks256 = ((M + 255) / 256) * ((N + 127) / 128);
    const int64_t blocks_wide = ((M + 127) / 128) * ((N + 255) / 256);
    if (dx && blocks_wide >= 256) return &kF32Tiles[3];
    if ((dw || kind == Kind::Fwd) && blocks256 >= 256) return &kF32Tiles[2];
    const int64_t blocks128 = ((M + 127) / 128) * ((N + 127) / 128);
    if (blocks128 >= 512) return &kF32Tiles[1];
    return &kF32Tiles[0];
}

int64_t tile_count(const GemmArgs& a, const Tile* t) { return ((a.M + t->bm - 1) / t->bm) * ((a.N + t->bn - 1) / t->bn); }

// The register-staged tile a direct fp32 tile falls back to when it cannot
// run a GEMM (same k order, so the same bits): the 256x128 and 128x256 twins,
// and 256x128 for the 256x256 tile.
const Tile* f32_register_twin(const Tile* t) {
    if (!t->bk) return t;
    if (t == &kF32Tiles[7]) return &kF32Tiles[0];
    return t == &kF32Tiles[5] ? &kF32Tiles[3] : &kF32Tiles[2];
}

// Direct-to-LDS tile for GEMM `kind` whose register tile is t, or null: the
// 256x256 tile for dX and dW on grids of at least 256 such tiles, the 64x64
// direct tile for a forward on the 64x64 register tile's small grids, else
// the twin of t.  The direct kernels take the plain forward, dX and dW (with or
// without the db side output): no masked operand, no dZ side output, K a
// multiple of 16 and vector-aligned operands (vec).  Measured on MI355X at
// 8192x4096x4096, alternating with the register kernels in one process
// (bit-identical outputs): forward 132.5 -> 139.0 TFLOP/s, dX 133 -> 138.5
// (its first fragment reads issued before the next tile's DMA; 141.0 on
// 256x256), dW with db 128.5 -> 134.6, without db 138.7 (139.6 on 256x256).
const Tile* f32_direct(Kind kind, const GemmArgs& a, const Tile* t, bool vec) {
    const bool plain = kind == Kind::Fwd || kind == Kind::Dx || kind == Kind::Dw;
    if (!plain || a.Amask || a.Bmask || a.dz || !vec || a.K < 16 || a.K % 16 != 0) return nullptr;
    if (t == &kF32Tiles[6]) return kind == Kind::Fwd ? nullptr : t;  // forced 256x256 (dX, dW only)
    if (t == &kF32Tiles[7]) return t;                                 // forced 64x64
    if (t->bk) t = f32_register_twin(t);  // forced twin: decide as for its register tile
    if (!f32_forced() && kind != Kind::Fwd && tile_count(a, &kF32Tiles[6]) >= 256) return &kF32Tiles[6];
    if (t == &kF32Tiles[2]) return &kF32Tiles[4];
    if (t == &kF32Tiles[3]) return &kF32Tiles[5];
    // A forward on at most 256 64x64 tiles (at most one round of blocks):
    // the 6-stage direct tile.  Measured on MI355X against the register
    // 64x64 tile, alternating in one process (bit-identical outputs):
    // 128x256x128 11.2 -> 9.8 us, 128x784x256 (split k) 12.8 -> 12.0,
    // 1024^3 35.1 -> 28.5, 512x4096x512 118.9 -> 92.4; on 1024 tiles
    // (2048x1024x2048) 85.1 -> 99.8, so larger grids keep the register tile.
    if (t == &kF32Tiles[0] && kind == Kind::Fwd && !f32_forced() && tile_count(a, t) <= 256) return &kF32Tiles[7];
    return nullptr;
}

const char* bf16_forced() {
    return !t_tile_bf16.empty() ? t_tile_bf16.c_str() : std::getenv("C3_HIP_GEMM_TILE_BF16");
}

const Tile* choose_bf16_tile(int64_t M, int64_t N) {
    const size_t nt = sizeof(kBf16Tiles) / sizeof(kBf16Tiles[0]);
    if (const char* forced = bf16_forced()) {
        if (const Tile* t = find_tile(kBf16Tiles, nt, forced)) return t;
    }
    const int64_t blocks128 = ((M + 127) / 128) * ((N + 127) / 128);
    if (blocks128 >= 256) return &kBf16Tiles[1];
    return &kBf16Tiles[0];
}

// Direct-to-LDS bf16 kernels (256x256 tiles): plain operands only (the
// backward masks are applied by the pre-pass), K a multiple of the tile's k
// depth, and a problem of at least 64 output tiles so the large tile fills
// the chip.
const Tile kBf16Direct[] = {{"d256w8", 256, 256, 512, 64, true},
                             {"d256rq", 256, 256, 256, 64, false},
                             {"d256pp", 256, 256, 512, 32, false},
                             {"d128w4", 128, 128, 256, 64, true},
                             {"d128w4s4", 128, 128, 256, 64, true},
                             {"d64w4", 64, 64, 256, 64, true}};

// K a multiple of the tile's k depth, or any K for a tile with a partial
// last k-tile (whose k-contiguous operands have K % 8 == 0 by the 16-byte
// vector rule checked before).
bool k_ok(const GemmArgs& a, const Tile* t) { return a.K % t->bk == 0 || t->ktail; }

bool direct_eligible(Kind kind, const GemmArgs& a, const Tile* t) {
    if (kind == Kind::DxMask || kind == Kind::DwMask || a.db != nullptr) return false;
    return a.K > 0 && a.M >= 8 && a.N >= 8 && k_ok(a, t);
}


// Split-K factor for direct tile t: the largest power of two S <= 32 with
// tiles * S <= max_blocks, each split at least min_k deep and a multiple of
// the tile's k depth, and an fp32 workspace of at most 256 MiB; 1 = no split.
int plan_split(const GemmArgs& a, const Tile* t, int64_t max_blocks, int64_t min_k) {
    const int64_t tiles = tile_count(a, t);
    int S = 1;
    for (int s = 2; s <= 32; s *= 2) {
        if (a.K % ((int64_t)s * t->bk) != 0 || a.K / s < min_k) break;
        if (tiles * s > max_blocks) break;
        if ((double)s * (double)a.M * (double)a.N * 4.0 > (double)(256u << 20)) break;
        S = s;
    }
    return S;
}

// Split plan of a forced direct tile: as the size heuristic would split it
// (fewer tiles than one block per CU), else 1.
int forced_split(const GemmArgs& a, const Tile* t) {
    // Blocks resident at once: two per CU for the 64 KiB tiles, else one.
    const bool two = std::strcmp(t->name, "d128w4") == 0 || std::strcmp(t->name, "d64w4") == 0;
    const int64_t per_wave = two ? 512 : 256;
    if (tile_count(a, t) >= per_wave / 2) return 1;
    return plan_split(a, t, per_wave, t->bm == 128 ? 256 : 512);
}

// Sets *unsupported when the calling thread forced a direct tile this
// problem cannot use; *split receives the split-K factor (1: none).
// Size heuristic (measured on MI355X over the 1024..16384 sweep shapes):
//  - 256x256 tiles when they give at least 256 blocks (one per CU), or, for
//    a weight gradient, reach 256 blocks with k split into parts at least
//    4096 deep;
//  - else 64x64 tiles (4 stages) when 128x128 tiles give fewer than 128
//    blocks, 64x64 tiles at least 256, and K <= 8192;
//  - else 128x128 tiles when they give at least 128 blocks, or for K >= 2048
//    when split-K brings them there; below 256 blocks the k range is split
//    into parts at least 512 deep, up to 512 blocks (two per CU); 128 to 256
//    blocks over K >= 2048 without a split take the 4-stage variant;
//  - else, for a weight gradient, 128x128 tiles when splits at least 256
//    deep reach 256 blocks;
//  - else the register-staged kernels (outputs smaller than 1024x1024).
const Tile* choose_bf16_direct(Kind kind, const GemmArgs& a, bool* unsupported, int* split) {
    *unsupported = false;
    *split = 1;
    const size_t nd = sizeof(kBf16Direct) / sizeof(kBf16Direct[0]);
    if (const char* forced = bf16_forced()) {
        const Tile* t = find_tile(kBf16Direct, nd, forced);
        if (!t) return nullptr;  // a register-staged tile was asked for
        if (direct_eligible(kind, a, t)) {
            *split = forced_split(a, t);
            return t;
        }
        *unsupported = !t_tile_bf16.empty();
        return nullptr;
    }
    if (kind == Kind::DxMask || kind == Kind::DwMask || a.db != nullptr) return nullptr;
    if (a.K == 0) return nullptr;
    if (a.M < 8 || a.N < 8) return nullptr;
    const Tile* big = find_tile(kBf16Direct, nd, "d256w8");
    const Tile* small = find_tile(kBf16Direct, nd, "d128w4");
    if (!k_ok(a, big) || !k_ok(a, small)) return nullptr;
    const int64_t tiles_b = tile_count(a, big);
    if (tiles_b >= 256) return big;
    // A weight gradient (k = the batch) on too few 256x256 tiles: split k
    // into parts at least 4096 deep until the splits fill the chip with one
    // block per CU.  Measured on MI355X for dW of the 4096 -> 1000 layer at
    // batch 16384: d128w4 on its 256 tiles (one block per CU) 229.5 us.
    // (Forward and dX keep the plans below, whose fp32 partials stay within
    // the no-allocation entry point's scratch.)
    if ((kind == Kind::Dw || kind == Kind::DwB) && tiles_b >= 32 && a.K >= 2 * 4096) {
        int S = 1;
        while (tiles_b * S < 256 && a.K / (2 * S) >= 4096 && a.K % (2 * S * big->bk) == 0 &&
               (double)(2 * S) * (double)a.M * (double)a.N * 4.0 <= (double)(256u << 20))
            S *= 2;
        if (tiles_b * S >= 256) {
            *split = S;
            return big;
        }
    }
    const int64_t tiles_s = tile_count(a, small);
    // Outputs too small for 128 128x128 tiles whose 64x64 tiles fill the chip
    // (a 1024x1024 output): 64x64 tiles, no split, up to k = 8192.  Measured
    // on MI355X at 1024x1024x1024 (forward / dX / dW): 8.3 / 7.4 / 7.5 us
    // against 18.2 / 10.8 / 18.7 for the register-staged 64x64 tile and the
    // split 128x128 dW; k = 4096: 19.5-20.3 us against 26.7-28.4 for split
    // 128x128 tiles; k = 8192 36.2 against 37.3.
    const Tile* tiny = find_tile(kBf16Direct, nd, "d64w4");
    if (tiles_s < 128 && tile_count(a, tiny) >= 256 && a.K <= 8192) return tiny;
    const int Ss = tiles_s >= 256 ? 1 : plan_split(a, small, 512, 512);  // 256 blocks: one per CU already
    if (tiles_s >= 128 || (a.K >= 2048 && tiles_s * Ss >= 128)) {
        // One block per CU over k >= 2048 (no split): four stages, three
        // tiles in flight.  Measured on MI355X on the 256-tile GEMMs of the
        // 4096 / 1024 sweep shapes with k = 4096: 44.0-46.5 us against
        // 46.6-50.1 for two stages; equal at k = 1024.
        if (Ss == 1 && tiles_s <= 256 && a.K >= 2048) return find_tile(kBf16Direct, nd, "d128w4s4");
        *split = Ss;
        return small;
    }
    // A weight gradient below that: 128x128 tiles with k split into parts at
    // least 256 deep when that reaches 256 blocks, where the register-staged
    // kernels read both (row-contiguous) operands slowly.  Measured on MI355X
    // at 1024x1024x1024: 18.5 us (4 splits) against 26.0 for the 64x64
    // register tile; the forward and dX stay on the register tiles (18.2 /
    // 10.9 us against 19.3 / 18.4).
    if (kind == Kind::Dw || kind == Kind::DwB) {
        const int S = plan_split(a, small, 512, 256);
        if (tiles_s * S >= 256) {
            *split = S;
            return small;
        }
    }
    return nullptr;
}

// Where a call's workspace came from: the caller's (nothing to free), the
// library's arena for the stream, or the stream-ordered allocator.
enum class WsHow { Caller, Arena, Stream };

// A workspace of `bytes` for one call: from ws when it has a base (capacity
// checked, nothing launched on failure), else from ws_alloc; *how tells
// release_workspace how to give it back.
int take_workspace(const Workspace* ws, size_t bytes, hipStream_t stream, void** p, WsHow* how, const char* what) {
    *how = WsHow::Caller;
    if (ws && ws->base) {
        if (bytes > ws->bytes)
            return set_error(C3HIP_ERR_TOO_LARGE, std::string(what) + " needs " + std::to_string(bytes) +
                                                      " bytes of workspace, more than the " + std::to_string(ws->bytes) +
                                                      " bytes given");
        *p = ws->base;
        return C3HIP_OK;
    }
    bool arena = false;
    const int rc = ws_alloc(bytes, stream, p, &arena, what);
    if (rc) return rc;
    *how = arena ? WsHow::Arena : WsHow::Stream;
    return C3HIP_OK;
}

int release_workspace(void* p, WsHow how, int rc, hipStream_t stream, const char* what) {
    if (how == WsHow::Caller) return rc;
    const int frc = ws_free(p, how == WsHow::Arena, stream, what);
    return rc != C3HIP_OK ? rc : frc;
}

// Split-K run of a plain bf16 GEMM on direct tile d: S block rows write fp32
// partial products into a workspace of the call [S, M, N]; the reduction
// adds them in split order and applies the kind's epilogue (forward: bias and
// activation, bf16 out; dW: fp32 out; the others: bf16 out).
int run_split(Kind kind, const GemmArgs& a0, const Tile* d, int S, hipStream_t stream, const Workspace* wsp) {
    // fp32-output kernel of the same operand layouts (FwdT: both k-contiguous, as dX).
    const char* kn = kind == Kind::Fwd                          ? "fwdf"
                     : (kind == Kind::Dx || kind == Kind::FwdT) ? "dxf"
                     : kind == Kind::TT                         ? "ttf"
                                                                : "dw";
    const bool fwd = kind == Kind::Fwd || kind == Kind::FwdT;
    float* ws = nullptr;
    WsHow how;
    const int64_t slice = a0.M * a0.N;
    int rc = take_workspace(wsp, (size_t)S * (size_t)slice * sizeof(float), stream, (void**)&ws, &how, "split-K");
    if (rc) return rc;
    GemmArgs g = a0;
    g.C = ws;
    g.ldc = a0.N;
    g.bias = nullptr;
    g.act = 0;
    g.split_k = a0.K / S;
    g.c_split = slice;
    char name[96];
    std::snprintf(name, sizeof(name), "c3_gemm_bf16_%s_%s", kn, d->name);
    const int64_t tiles = tile_count(a0, d);
    void* args[] = {&g};
    rc = launch(name, dim3((unsigned)tiles, (unsigned)S), dim3(d->threads), args, stream);
    if (rc == C3HIP_OK) {
        SplitReduceArgs r{};
        r.ws = ws;
        r.C = a0.C;
        r.bias = fwd ? a0.bias : nullptr;
        r.M = a0.M;
        r.N = a0.N;
        r.ldc = a0.ldc;
        r.slice = slice;
        r.S = S;
        r.act = fwd ? a0.act : 0;
        r.out_bf16 = kind == Kind::Dw ? 0 : 1;
        const int64_t threads = a0.M * ((a0.N + 3) / 4);
        void* rargs[] = {&r};
        rc = launch("c3_splitk_reduce", dim3((unsigned)((threads + 255) / 256)), dim3(256), rargs, stream);
    }
    return release_workspace(ws, how, rc, stream, "split-K");
}

// bf16 kernels always move 16-byte vectors (8 elements): the contiguous
// extent and the leading dimension must be multiples of 8.
bool bf16_vec_ok(bool kc, int64_t rows, int64_t k, int64_t ld, const void* p, const void* pm) {
    if (ld % 8 != 0) return false;
    if (kc ? (k % 8 != 0) : (rows % 8 != 0)) return false;
    return aligned16(p) && aligned16(pm);
}

// Can an operand use 16-byte vector loads?  kc: k is its contiguous index.
bool vec_ok(bool kc, int64_t rows, int64_t k, int64_t ld, const void* p, const void* pm) {
    if (ld % 4 != 0) return false;
    if (kc ? (k % 4 != 0) : (rows % 4 != 0)) return false;
    return aligned16(p) && aligned16(pm);
}

// fp32 split-K for a small grid over a long k range (a train step's first
// layer at batch 128: 8 tiles of 64x64 over K = 784): the 64x64 kernel on
// fewer than 32 tiles with K >= 512 and no db side output splits k into
// 16-aligned parts at least 128 deep, up to 256 blocks; 0 = no split.  A
// forced tile never splits.
// Kernel name of register tile t for a GEMM over K: the 64x64 tile's
// all-k-at-once kernels (t64x64k: every k-tile's loads issued together, one
// memory round trip) for K <= 128 with vector-aligned operands, else the
// tile's k loop.  Same operations in the same order, so the same bits.
// Measured on MI355X in the 784-256-128-10 train step: layer 2's one-launch
// backward 11.6 -> 10.6 us, layer 1's dW 11.4 -> 10.4; the scalar-load
// kernels (layer 3, N = 10) were slower in that form and keep the loop.
const char* f32_reg_name(const Tile* t, int64_t K, bool vec) {
    return t == &kF32Tiles[0] && K <= 128 && vec ? "t64x64k" : t->name;
}

int plan_split_f32(const GemmArgs& a, const Tile* t) {
    if (!t_tile_f32.empty() || std::getenv("C3_HIP_GEMM_TILE")) return 0;
    if (t->bm != 64 || a.db != nullptr || a.dz != nullptr || a.K < 512) return 0;
    const int64_t tiles = tile_count(a, t);
    if (tiles >= 32) return 0;
    int64_t S = std::min<int64_t>(256 / tiles, a.K / 128);
    if ((double)S * (double)a.M * (double)a.N * 4.0 > (double)(256u << 20)) S = (256 << 20) / (a.M * a.N * 4);
    return S >= 2 ? (int)S : 0;
}

int run_split_f32(Kind kind, const GemmArgs& a0, const Tile* t, int S, bool vec, hipStream_t stream,
                  const Workspace* wsp) {
    const int64_t split_k = ((a0.K + S - 1) / S + 15) / 16 * 16;
    S = (int)((a0.K + split_k - 1) / split_k);
    const int64_t slice = a0.M * a0.N;
    float* ws = nullptr;
    WsHow how;
    int rc = take_workspace(wsp, (size_t)S * (size_t)slice * sizeof(float), stream, (void**)&ws, &how, "split-K");
    if (rc) return rc;
    GemmArgs g = a0;
    g.C = ws;
    g.ldc = a0.N;
    g.bias = nullptr;
    g.act = 0;
    g.split_k = split_k;
    g.c_split = slice;
    char name[96];
    if (t->bk) std::snprintf(name, sizeof(name), "c3_gemm_f32_%s_%s", kind_name(kind), t->name);
    else std::snprintf(name, sizeof(name), "c3_gemm_f32_%s_%s_%s", kind_name(kind), f32_reg_name(t, split_k, vec), vec ? "v" : "s");
    void* args[] = {&g};
    rc = launch(name, dim3((unsigned)tile_count(a0, t), (unsigned)S), dim3(t->threads), args, stream);
    if (rc == C3HIP_OK) {
        SplitReduceArgs r{};
        r.ws = ws;
        r.C = a0.C;
        r.bias = a0.bias;
        r.M = a0.M;
        r.N = a0.N;
        r.ldc = a0.ldc;
        r.slice = slice;
        r.S = S;
        r.act = a0.act;
        r.out_bf16 = 0;
        const int64_t threads = a0.M * ((a0.N + 3) / 4);
        void* rargs[] = {&r};
        rc = launch("c3_splitk_reduce", dim3((unsigned)((threads + 255) / 256)), dim3(256), rargs, stream);
    }
    return release_workspace(ws, how, rc, stream, "split-K");
}

int run_gemm(int dtype, Kind kind, const GemmArgs& a0, bool a_kc, bool b_kc, hipStream_t stream,
             const Workspace* ws = nullptr) {
    GemmArgs a = a0;
    if (a.M == 0 || a.N == 0) return C3HIP_OK;
    if (dtype == C3HIP_BF16) {
        if (!bf16_vec_ok(a_kc, a.M, a.K, a.lda, a.A, a.Amask) || !bf16_vec_ok(b_kc, a.N, a.K, a.ldb, a.B, a.Bmask))
            return set_error(C3HIP_ERR_UNSUPPORTED,
                             "bf16 GEMM needs 16-byte aligned operands and contiguous extents that are multiples of 8");
        bool unsupported = false;
        int split = 1;
        const Tile* d = choose_bf16_direct(kind, a, &unsupported, &split);
        if (unsupported)
            return set_error(C3HIP_ERR_UNSUPPORTED, std::string("tile ") + t_tile_bf16 +
                                                        " cannot run this GEMM (masked operand, db side output, "
                                                        "K not a multiple of its k depth, or M or N below 8)");
        if (d && split > 1) return run_split(kind, a, d, split, stream, ws);
        if (!d && kind == Kind::FwdT) return set_error(C3HIP_ERR_UNSUPPORTED, "transposed-W forward needs a direct tile");
        if (d) {
            char name[96];
            std::snprintf(name, sizeof(name), "c3_gemm_bf16_%s_%s", kind_name(kind), d->name);
            const int64_t blocks = tile_count(a, d);
            void* args[] = {&a};
            return launch(name, dim3((unsigned)blocks), dim3(d->threads), args, stream);
        }
        const Tile* t = choose_bf16_tile(a.M, a.N);
        char name[96];
        std::snprintf(name, sizeof(name), "c3_gemm_bf16_%s_%s", kind_name(kind), t->name);
        const int64_t blocks = ((a.M + t->bm - 1) / t->bm) * ((a.N + t->bn - 1) / t->bn);
        if (blocks > 0x7fffffff) return set_error(C3HIP_ERR_TOO_LARGE, "GEMM grid too large");
        void* args[] = {&a};
        return launch(name, dim3((unsigned)blocks), dim3(t->threads), args, stream);
    }
    const Tile* t = choose_f32_tile(kind, a.M, a.N);
    const bool vec = vec_ok(a_kc, a.M, a.K, a.lda, a.A, a.Amask) && vec_ok(b_kc, a.N, a.K, a.ldb, a.B, a.Bmask);
    // A forced register tile runs as itself; the size heuristic's big tiles
    // and a forced direct tile run direct where f32_direct allows (else the
    // direct tile's register twin).
    const bool forced_reg = f32_forced() && !t->bk;
    if (const Tile* d = forced_reg ? nullptr : f32_direct(kind, a, t, vec)) {
        if (d == &kF32Tiles[7])
            if (const int S = plan_split_f32(a, &kF32Tiles[0])) return run_split_f32(kind, a, d, S, vec, stream, ws);
        char name[96];
        std::snprintf(name, sizeof(name), "c3_gemm_f32_%s_%s", kind_name(kind), d->name);
        const int64_t blocks = tile_count(a, d);
        if (blocks > 0x7fffffff) return set_error(C3HIP_ERR_TOO_LARGE, "GEMM grid too large");
        void* args[] = {&a};
        return launch(name, dim3((unsigned)blocks), dim3(d->threads), args, stream);
    }
    t = f32_register_twin(t);
    if (const int S = plan_split_f32(a, t)) return run_split_f32(kind, a, t, S, vec, stream, ws);
    char name[96];
    std::snprintf(name, sizeof(name), "c3_gemm_f32_%s_%s_%s", kind_name(kind), f32_reg_name(t, a.K, vec), vec ? "v" : "s");
    const int64_t blocks = ((a.M + t->bm - 1) / t->bm) * ((a.N + t->bn - 1) / t->bn);
    if (blocks > 0x7fffffff) return set_error(C3HIP_ERR_TOO_LARGE, "GEMM grid too large");
    void* args[] = {&a};
    return launch(name, dim3((unsigned)blocks), dim3(t->threads), args, stream);
}

// bf16 forward with W transposed first: both GEMM operands are then
// k-contiguous and read with ds_read_b128 instead of transposed LDS reads.
// Same tile, split and k order as the plain forward, so the same bits.
// Opt-in (C3_HIP_BF16_WT=1, whenever a direct tile runs the forward): measured
// on MI355X with the transpose included it gains 4% at 8192x4096x4096 and
// loses 1.5% at 16384x4096x8192 and 27% at 4096x1024x4096, so the size
// heuristic never picks it.
bool bf16_fwd_transposed(const GemmArgs& a) {
    const char* env = std::getenv("C3_HIP_BF16_WT");
    if (!env || env[0] != '1') return false;
    if (a.K % 8 != 0 || a.N % 8 != 0 || !aligned16(a.A) || !aligned16(a.B)) return false;
    if ((a.K + 63) / 64 > 65535 || (a.N + 63) / 64 > 0x7fffffff) return false;  // transpose grid
    bool unsupported = false;
    int split = 1;
    return choose_bf16_direct(Kind::Fwd, a, &unsupported, &split) != nullptr;
}

int linear_fwd_wt(const GemmArgs& a0, hipStream_t stream) {
    void* wt = nullptr;
    WsHow how;
    if (int rc0 = take_workspace(nullptr, (size_t)(a0.K * a0.N) * 2, stream, &wt, &how, "W^T")) return rc0;
    const void* w = a0.B;
    int64_t R = a0.K, Cc = a0.N;
    void* targs[] = {(void*)&w, &wt, &R, &Cc};
    int rc = launch("c3_transpose_bf16", dim3((unsigned)((Cc + 63) / 64), (unsigned)((R + 63) / 64)), dim3(256), targs,
                    stream);
    if (rc == C3HIP_OK) {
        GemmArgs a = a0;
        a.B = wt;
        a.ldb = a0.K;
        rc = run_gemm(C3HIP_BF16, Kind::FwdT, a, true, true, stream);
    }
    return release_workspace(wt, how, rc, stream, "W^T");
}

int check_elems(const char* what, int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0) return set_error(C3HIP_ERR_INVALID, std::string(what) + ": negative dimension");
    if (cols > 0 && rows > (kMaxElems32 - 1) / cols)
        return set_error(C3HIP_ERR_TOO_LARGE, std::string(what) + ": more than 2^32 elements");
    return C3HIP_OK;
}

int check_dtype(int dtype) {
    if (dtype != C3HIP_F32 && dtype != C3HIP_BF16) return set_error(C3HIP_ERR_INVALID, "unknown dtype " + std::to_string(dtype));
    return C3HIP_OK;
}

// Launch shape of a column-sum pass over M rows of `units` column units (a
// column, or an 8-column vector for bf16): blocks of vb units x 256 / vb row
// lanes, about 256 K threads in all, each adding at least 4 rows.
struct ColGeom {
    int vb;
    unsigned gx;
    int64_t rows_per_chunk, nchunks;
};

ColGeom col_geom(int64_t M, int64_t units) {
    ColGeom g{};
    g.vb = units > 128 ? 256 : units > 64 ? 128 : 64;
    const int64_t rb = 256 / g.vb;
    g.gx = (unsigned)((units + g.vb - 1) / g.vb);
    const int64_t rows_per_thread = std::max<int64_t>(4, (M * units + (1 << 18) - 1) >> 18);
    g.rows_per_chunk = std::max<int64_t>(1, rows_per_thread * rb);
    g.nchunks = std::max<int64_t>(1, (M + g.rows_per_chunk - 1) / g.rows_per_chunk);
    return g;
}

// Adds the nchunks partial rows of part [nchunks, N] into out[N].
int colsum_final(const float* part, float* out, int64_t nchunks, int64_t N, hipStream_t stream) {
    void* args[] = {(void*)&part, (void*)&out, &nchunks, &N};
    return launch("c3_colsum_final_f32", dim3((unsigned)((N + 63) / 64)), dim3(512), args, stream);
}

// Column sums of (optionally masked) fp32 [M,N] into out[N]: one pass when
// one chunk covers M, else per-chunk partials in a workspace of the call.
int colsum(const float* in, const float* mask, float* out, int64_t M, int64_t N, hipStream_t stream) {
    if (N == 0) return C3HIP_OK;
    ColGeom g = col_geom(M, N);
    int64_t rows_per_chunk = g.rows_per_chunk, nchunks = g.nchunks;
    int vb = g.vb;
    const char* pname = "c3_colsum_partial_f32";
    if (nchunks == 1) {
        void* args[] = {(void*)&in, (void*)&mask, (void*)&out, &M, &N, &rows_per_chunk, &vb};
        return launch(pname, dim3(g.gx, 1), dim3(256), args, stream);
    }
    float* part = nullptr;
    WsHow how;
    if (int rc0 = take_workspace(nullptr, (size_t)(nchunks * N) * sizeof(float), stream, (void**)&part, &how,
                                 "column-sum partials"))
        return rc0;
    void* args1[] = {(void*)&in, (void*)&mask, (void*)&part, &M, &N, &rows_per_chunk, &vb};
    int rc = launch(pname, dim3(g.gx, (unsigned)nchunks), dim3(256), args1, stream);
    if (rc == C3HIP_OK) rc = colsum_final(part, out, nchunks, N, stream);
    return release_workspace(part, how, rc, stream, "column-sum partials");
}

// Arguments of c3_gemm_bf16_bwd_<tile> (gemm_bf16.hip).
struct Bf16BwdArgs {
    GemmArgs dx;
    GemmArgs dw;
    const float* part;
    float* db;
    int64_t nchunks;
    int nx, nw;
};

// Whether the size heuristic runs both GEMMs of a bf16 layer backward (ax:
// dX, aw: dW) on direct tiles without a split and a one-launch kernel
// (c3_gemm_bf16_bwd_<dX tile>[_<dW tile>]) exists for the two tiles: the
// same tile, or the 64x64 and 128x128 tiles (same block size and LDS); no
// tile forced.  That launch also runs the bias gradient's final pass.
// Measured on MI355X against the separate launches, alternating in one
// process over the 27 sweep shapes (bit-identical outputs): 1024^3
// backward 24.5 -> 19.5 us, 1024x4096x1024 44.2 -> 33.4, 4096^3 270 -> 262;
// the others within 1%.
// Where the heuristic puts dX and dW on different 128x128 / 256x256 tiles,
// or both on the four-stage 128x128 tile, both run on the two-stage 128x128
// tile in one launch (two blocks per CU), up to 4608 such tiles in all (the
// largest pair measured; larger pairs keep the separate launches).
// Measured alternately against the separate launches (backward with its
// pre-pass, bit-identical): 1024x4096x4096 107.4 -> 90.2 us, 1024x4096x8192
// 189.2 -> 158.4, 1024x8192x4096 166.0 -> 151.7, 1024x8192x8192 336.1 ->
// 323.6, 4096x1024x8192 189.5 -> 168.1, 4096x4096x1024 100.9 -> 94.7,
// 4096x8192x1024 159.5 -> 159.2; the four-stage tile for both was slower
// than the separate launches there.  Against the four-stage one-launch pair
// (fwd + bwd step, four alternating rounds): 4096x1024x4096 629-722 ->
// 740-800 TFLOP/s, 2048^3 509-599 -> 610-670.
bool bf16_bwd_pair_tiles(const GemmArgs& ax, const GemmArgs& aw, const Tile** tx, const Tile** tw) {
    if (bf16_forced()) return false;
    if (!bf16_vec_ok(true, ax.M, ax.K, ax.lda, ax.A, nullptr) || !bf16_vec_ok(true, ax.N, ax.K, ax.ldb, ax.B, nullptr) ||
        !bf16_vec_ok(false, aw.M, aw.K, aw.lda, aw.A, nullptr) || !bf16_vec_ok(false, aw.N, aw.K, aw.ldb, aw.B, nullptr))
        return false;
    bool unsupported = false;
    int sx = 1, sw = 1;
    *tx = choose_bf16_direct(Kind::Dx, ax, &unsupported, &sx);
    *tw = choose_bf16_direct(Kind::Dw, aw, &unsupported, &sw);
    if (!*tx || !*tw || sx != 1 || sw != 1) return false;
    auto is = [](const Tile* t, const char* n) { return std::strcmp(t->name, n) == 0; };
    const bool same = *tx == *tw && (is(*tx, "d256w8") || is(*tx, "d128w4") || is(*tx, "d64w4"));
    const bool mixed = (is(*tx, "d64w4") && is(*tw, "d128w4")) || (is(*tx, "d128w4") && is(*tw, "d64w4"));
    if (!same && !mixed) {
        auto direct = [&](const Tile* t) { return is(t, "d256w8") || is(t, "d128w4") || is(t, "d128w4s4"); };
        if (!direct(*tx) || !direct(*tw)) return false;
        // choose_bf16_direct returned a direct tile for each, so both passed
        // k_ok for the 128x128 tile too.
        const Tile* t = find_tile(kBf16Direct, sizeof(kBf16Direct) / sizeof(kBf16Direct[0]), "d128w4");
        if (!t || tile_count(ax, t) + tile_count(aw, t) > 4608) return false;
        *tx = *tw = t;
    }
    return tile_count(ax, *tx) + tile_count(aw, *tw) + (aw.N + 63) / 64 <= 0x7fffffff;
}

// Backward through a pre-pass: one pass forms dZ = act'(Y) * dY (in the
// layer's dtype, a workspace of the call) together with the per-chunk column
// sums for db, then dX and dW run as plain GEMMs on dZ.  Used for every bf16
// backward (the direct-to-LDS kernels cannot apply a mask while loading), for
// the fp32 sigmoid/tanh backward (the fp32 GEMMs fuse only the ReLU mask), and
// for the fp32 ReLU backward whose plain dX and dW run direct (f32_bwd_direct).
// Without an activation, dZ is dY itself.  bf16 dX, dW and the db final
// pass go in one launch where bf16_bwd_pair_tiles allows.
int linear_bwd_prepass(int dtype, const void* X, const void* W, const void* Y, const void* dY, void* dX, float* dW,
                       float* db, int64_t M, int64_t K, int64_t N, int act, hipStream_t stream) {
    const size_t esz = dtype == C3HIP_BF16 ? 2 : 4;
    if (M == 0 || N == 0) {
        if (db && N > 0) {
            hipError_t e = hipMemsetAsync(db, 0, (size_t)N * sizeof(float), stream);
            if (e != hipSuccess) return set_error(C3HIP_ERR_HIP, std::string("hipMemsetAsync: ") + hipGetErrorString(e));
        }
        if (dW && K > 0 && N > 0) {
            hipError_t e = hipMemsetAsync(dW, 0, (size_t)(K * N) * sizeof(float), stream);
            if (e != hipSuccess) return set_error(C3HIP_ERR_HIP, std::string("hipMemsetAsync: ") + hipGetErrorString(e));
        }
        if (dX && M > 0 && K > 0) {
            hipError_t e = hipMemsetAsync(dX, 0, (size_t)(M * K) * esz, stream);
            if (e != hipSuccess) return set_error(C3HIP_ERR_HIP, std::string("hipMemsetAsync: ") + hipGetErrorString(e));
        }
        return C3HIP_OK;
    }
    if (dtype == C3HIP_BF16 && (N % 8 != 0 || !aligned16(Y) || !aligned16(dY)))
        return set_error(C3HIP_ERR_UNSUPPORTED, "bf16 backward needs N % 8 == 0 and 16-byte aligned Y, dY");
    const bool need_dz = act != C3HIP_ACT_NONE && (dX || dW);
    // fp32 rows of 16-byte vectors take the vector pre-pass (4 columns per thread).
    const bool f32v = dtype == C3HIP_F32 && N % 4 == 0 && aligned16(Y) && aligned16(dY);
    const ColGeom g = col_geom(M, dtype == C3HIP_BF16 ? N / 8 : f32v ? N / 4 : N);
    int64_t nchunks = g.nchunks, rows_per_chunk = g.rows_per_chunk;
    int vb = g.vb;
    void* dz = nullptr;
    float* part = nullptr;
    WsHow dz_how = WsHow::Caller, part_how = WsHow::Caller;
    int rc = C3HIP_OK;
    if (need_dz && (rc = take_workspace(nullptr, (size_t)(M * N) * esz, stream, &dz, &dz_how, "dZ"))) return rc;
    if (db && nchunks > 1 &&
        (rc = take_workspace(nullptr, (size_t)(nchunks * N) * sizeof(float), stream, (void**)&part, &part_how,
                             "column-sum partials"))) {
        if (dz) (void)release_workspace(dz, dz_how, rc, stream, "dZ");
        return rc;
    }
    const void* dzp = need_dz ? dz : dY;
    GemmArgs ax{};
    ax.A = dzp; ax.B = W; ax.C = dX;
    ax.M = M; ax.N = K; ax.K = N;
    ax.lda = N; ax.ldb = N; ax.ldc = K;
    GemmArgs aw{};
    aw.A = X; aw.B = dzp; aw.C = dW;
    aw.M = K; aw.N = N; aw.K = M;
    aw.lda = K; aw.ldb = N; aw.ldc = N;
    const Tile *px = nullptr, *pw = nullptr;
    const bool pair = dtype == C3HIP_BF16 && dX && dW && K > 0 && bf16_bwd_pair_tiles(ax, aw, &px, &pw);
    if (need_dz || db) {
        float* part_out = db ? (nchunks > 1 ? part : db) : nullptr;
        int act_i = act;
        void* args[] = {(void*)&Y, (void*)&dY, &dz, &part_out, &M, &N, &rows_per_chunk, &act_i, &vb};
        rc = launch(dtype == C3HIP_BF16 ? "c3_dz_colsum_bf16" : f32v ? "c3_dz_colsum_f32_v" : "c3_dz_colsum_f32",
                    dim3(g.gx, (unsigned)nchunks), dim3(256), args, stream);
        if (rc == C3HIP_OK && db && nchunks > 1 && !pair) rc = colsum_final(part, db, nchunks, N, stream);
    }
    if (rc == C3HIP_OK && pair) {
        Bf16BwdArgs p{};
        p.dx = ax;
        p.dw = aw;
        p.nx = (int)tile_count(ax, px);
        p.nw = (int)tile_count(aw, pw);
        const int64_t nf = db && nchunks > 1 ? (N + 63) / 64 : 0;
        p.part = part;
        p.db = db;
        p.nchunks = nchunks;
        char name[64];
        if (px == pw) std::snprintf(name, sizeof(name), "c3_gemm_bf16_bwd_%s", px->name);
        else std::snprintf(name, sizeof(name), "c3_gemm_bf16_bwd_%s_%s", px->name, pw->name);
        void* args[] = {&p};
        rc = launch(name, dim3((unsigned)(p.nx + p.nw + nf)), dim3(px->threads), args, stream);
    } else {
        if (rc == C3HIP_OK && dX) rc = run_gemm(dtype, Kind::Dx, ax, true, true, stream);
        if (rc == C3HIP_OK && dW) rc = run_gemm(dtype, Kind::Dw, aw, false, false, stream);
    }
    if (part) rc = release_workspace(part, part_how, rc, stream, "column-sum partials");
    if (dz) rc = release_workspace(dz, dz_how, rc, stream, "dZ");
    return rc;
}

}  // namespace

int linear_fwd(int dtype, const void* X, const void* W, const float* b, void* Y, int64_t M, int64_t K, int64_t N,
               int act, hipStream_t stream, const Workspace* ws) {
    int rc = check_dtype(dtype);
    if (rc) return rc;
    if (act < C3HIP_ACT_NONE || act > C3HIP_ACT_TANH) return set_error(C3HIP_ERR_INVALID, "unknown act");
    if ((rc = check_elems("X", M, K)) || (rc = check_elems("W", K, N)) || (rc = check_elems("Y", M, N))) return rc;
    if (M > 0 && N > 0 && (!Y || (K > 0 && (!X || !W)))) return set_error(C3HIP_ERR_INVALID, "null pointer");
    GemmArgs a{};
    a.A = X; a.B = W; a.C = Y; a.bias = b;
    a.M = M; a.N = N; a.K = K;
    a.lda = K; a.ldb = N; a.ldc = N;
    a.act = act;
    if (!(ws && ws->base) && dtype == C3HIP_BF16 && M > 0 && N > 0 && K > 0 && bf16_fwd_transposed(a))
        return linear_fwd_wt(a, stream);
    return run_gemm(dtype, Kind::Fwd, a, true, false, stream, ws);
}

}  // namespace c3hip

using namespace c3hip;

extern "C" {

int c3hip_elementwise(int op, int dtype, const void* a, const void* b, float alpha, void* out, int64_t n,
                      int64_t bmod, void* stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    const char* nm = ew_name(op);
    if (!nm) return set_error(C3HIP_ERR_INVALID, "unknown elementwise op " + std::to_string(op));
    int rc = check_dtype(dtype);
    if (rc) return rc;
    if (dtype != C3HIP_F32) return set_error(C3HIP_ERR_UNSUPPORTED, "elementwise ops take fp32 only");
    if (n < 0) return set_error(C3HIP_ERR_INVALID, "n < 0");
    if (n == 0) return C3HIP_OK;
    const bool binary = ew_is_binary(op);
    if (!a || !out || (binary && !b)) return set_error(C3HIP_ERR_INVALID, "null pointer");
    if (bmod == n) bmod = 0;
    if (!binary && bmod > 0) bmod = 0;
    char name[64];
    const bool vec = (n % 4 == 0) && aligned16(a) && aligned16(out) && (bmod >= 0) &&
                     (!binary || (aligned16(b) && (bmod == 0 || bmod % 4 == 0)));
    if (vec) {
        std::snprintf(name, sizeof(name), "c3_ew_%s_f32_v", nm);
        int64_t n4 = n / 4, bmod4 = bmod / 4;
        const int64_t blocks = (n4 + kEwVecThreads - 1) / kEwVecThreads;  // one vector per thread
        if (blocks > 0x7fffffff) return set_error(C3HIP_ERR_TOO_LARGE, "elementwise grid too large");
        void* args[] = {(void*)&a, (void*)&b, &alpha, &out, &n4, &bmod4};
        return launch(name, dim3((unsigned)blocks), dim3(kEwVecThreads), args, stream);
    }
    std::snprintf(name, sizeof(name), "c3_ew_%s_f32_s", nm);
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 1 << 16);
    void* args[] = {(void*)&a, (void*)&b, &alpha, &out, &n, &bmod};
    return launch(name, dim3((unsigned)blocks), dim3(256), args, stream);
}

int c3hip_elementwise3(int op, int dtype, const void* a, const void* b, const void* c, void* out, int64_t n,
                       void* stream) {
    clear_error();
    if (op != C3HIP_EW3_DIV_BWD_B) return set_error(C3HIP_ERR_INVALID, "unknown three-input op " + std::to_string(op));
    int rc = check_dtype(dtype);
    if (rc) return rc;
    if (dtype != C3HIP_F32) return set_error(C3HIP_ERR_UNSUPPORTED, "elementwise ops take fp32 only");
    if (n < 0) return set_error(C3HIP_ERR_INVALID, "n < 0");
    if (n == 0) return C3HIP_OK;
    if (!a || !b || !c || !out) return set_error(C3HIP_ERR_INVALID, "null pointer");
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 1 << 16);
    void* args[] = {(void*)&a, (void*)&b, (void*)&c, &out, &n};
    return launch("c3_ew3_div_bwd_b_f32", dim3((unsigned)blocks), dim3(256), args, (hipStream_t)stream);
}

int c3hip_set_gemm_tile(int dtype, const char* name) {
    clear_error();
    int rc = check_dtype(dtype);
    if (rc) return rc;
    std::string& slot = dtype == C3HIP_BF16 ? t_tile_bf16 : t_tile_f32;
    if (!name || !*name) {
        slot.clear();
        return C3HIP_OK;
    }
    const bool known =
        dtype == C3HIP_BF16
            ? (find_tile(kBf16Tiles, sizeof(kBf16Tiles) / sizeof(kBf16Tiles[0]), name) ||
               find_tile(kBf16Direct, sizeof(kBf16Direct) / sizeof(kBf16Direct[0]), name))
            : find_tile(kF32Tiles, sizeof(kF32Tiles) / sizeof(kF32Tiles[0]), name) != nullptr;
    if (!known) return set_error(C3HIP_ERR_INVALID, std::string("unknown GEMM tile ") + name);
    slot = name;
    return C3HIP_OK;
}

int c3hip_gemm_tile_names(int dtype, char* buf, size_t buflen) {
    clear_error();
    int rc = check_dtype(dtype);
    if (rc) return rc;
    std::string names;
    auto add = [&](const Tile* tiles, size_t n) {
        for (size_t i = 0; i < n; ++i) names += (names.empty() ? "" : ",") + std::string(tiles[i].name);
    };
    if (dtype == C3HIP_BF16) {
        add(kBf16Tiles, sizeof(kBf16Tiles) / sizeof(kBf16Tiles[0]));
        add(kBf16Direct, sizeof(kBf16Direct) / sizeof(kBf16Direct[0]));
    } else {
        add(kF32Tiles, sizeof(kF32Tiles) / sizeof(kF32Tiles[0]));
    }
    if (!buf || buflen < names.size() + 1) return set_error(C3HIP_ERR_INVALID, "buffer too small");
    std::memcpy(buf, names.c_str(), names.size() + 1);
    return C3HIP_OK;
}

int c3hip_backward_chain(int dtype, const void* grad, const void* const* x, const int* nodes, int num_nodes,
                         void* const* outs, int64_t n, void* stream) {
    clear_error();
    int rc = check_dtype(dtype);
    if (rc) return rc;
    if (dtype != C3HIP_F32) return set_error(C3HIP_ERR_UNSUPPORTED, "backward chains take fp32 only");
    if (num_nodes < 1 || num_nodes > kChainMaxNodes)
        return set_error(C3HIP_ERR_INVALID, "num_nodes must be 1.." + std::to_string(kChainMaxNodes));
    if (!nodes) return set_error(C3HIP_ERR_INVALID, "null node list");
    for (int k = 0; k < num_nodes; ++k)
        if (nodes[k] < C3HIP_CHAIN_RELU || nodes[k] > C3HIP_CHAIN_NEG)
            return set_error(C3HIP_ERR_INVALID, "unknown chain node " + std::to_string(nodes[k]));
    if (n < 0) return set_error(C3HIP_ERR_INVALID, "n < 0");
    if (n == 0) return C3HIP_OK;
    if (!grad || !x || !outs) return set_error(C3HIP_ERR_INVALID, "null pointer");
    ChainArgs p{};
    p.g = static_cast<const float*>(grad);
    p.w = num_nodes;
    bool vec = n % 4 == 0 && aligned16(grad);
    for (int k = 0; k < num_nodes; ++k) {
        if (nodes[k] != C3HIP_CHAIN_NEG && !x[k]) return set_error(C3HIP_ERR_INVALID, "null forward input");
        p.node[k] = nodes[k];
        p.x[k] = nodes[k] == C3HIP_CHAIN_NEG ? nullptr : static_cast<const float*>(x[k]);
        p.out[k] = static_cast<float*>(outs[k]);
        vec = vec && aligned16(p.x[k]) && aligned16(p.out[k]);
    }
    void* args[] = {&p};
    if (vec) {
        p.n = n / 4;
        const int64_t blocks = (p.n + kEwVecThreads - 1) / kEwVecThreads;  // one float4 per thread
        if (blocks > 0x7fffffff) return set_error(C3HIP_ERR_TOO_LARGE, "chain grid too large");
        return launch("c3_bwd_chain_f32_v", dim3((unsigned)blocks), dim3(kEwVecThreads), args, (hipStream_t)stream);
    }
    p.n = n;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 1 << 16);
    return launch("c3_bwd_chain_f32_s", dim3((unsigned)blocks), dim3(256), args, (hipStream_t)stream);
}

int c3hip_matmul(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t K, int64_t N, int transA,
                 int transB, void* stream) {
    clear_error();
    int rc = check_dtype(dtype);
    if (rc) return rc;
    if ((rc = check_elems("A", M, K)) || (rc = check_elems("B", K, N)) || (rc = check_elems("C", M, N))) return rc;
    if (M > 0 && N > 0 && (!C || (K > 0 && (!A || !B)))) return set_error(C3HIP_ERR_INVALID, "null pointer");
    GemmArgs a{};
    a.A = A; a.B = B; a.C = C;
    a.M = M; a.N = N; a.K = K;
    a.lda = transA ? M : K;
    a.ldb = transB ? K : N;
    a.ldc = N;
    a.act = C3HIP_ACT_NONE;
    const bool a_kc = !transA, b_kc = transB != 0;
    Kind kind = !transA ? (transB ? Kind::Dx : Kind::Fwd) : (transB ? Kind::TT : Kind::Dw);
    // bf16 matmul writes bf16 in every case; the dW kind writes fp32 for the
    // weight gradient, so the plain A^T.B product uses its bf16-output twin.
    if (dtype == C3HIP_BF16 && kind == Kind::Dw) kind = Kind::DwB;
    return run_gemm(dtype, kind, a, a_kc, b_kc, (hipStream_t)stream);
}

int c3hip_linear_fwd(int dtype, const void* X, const void* W, const float* b, void* Y, int64_t M, int64_t K,
                     int64_t N, int act, void* stream) {
    clear_error();
    return c3hip::linear_fwd(dtype, X, W, b, Y, M, K, N, act, (hipStream_t)stream, nullptr);
}

// fp32 ReLU backward through the vector pre-pass (dZ and the db partials in
// one stream over dY and Y) and plain direct-to-LDS dX and dW on dZ, when both
// plain GEMMs of this shape would run direct: measured on MI355X at
// 8192x4096x4096 the three launches take 65 + 1985 + 1980 us against 2165 +
// 2146 us for the masked dX that writes dZ and dW + db on it.  Decided on the
// shape and alignment alone, not on which of dX, dW, db are asked for, so a
// call for a subset of them returns the bits of the full call (db is then
// always the pre-pass column sum).
bool f32_bwd_direct(const GemmArgs& ax, const GemmArgs& aw, const void* Y, const void* dY) {
    if (ax.K % 4 != 0 || !aligned16(Y) || !aligned16(dY)) return false;
    const auto direct = [](Kind kind, GemmArgs a, bool a_kc, bool b_kc) {
        a.Amask = a.Bmask = nullptr;
        a.db = nullptr;
        const bool vec = vec_ok(a_kc, a.M, a.K, a.lda, a.A, nullptr) && vec_ok(b_kc, a.N, a.K, a.ldb, a.B, nullptr);
        if (f32_forced() && !choose_f32_tile(kind, a.M, a.N)->bk) return false;
        return f32_direct(kind, a, choose_f32_tile(kind, a.M, a.N), vec) != nullptr;
    };
    return direct(Kind::Dx, ax, true, true) && direct(Kind::Dw, aw, false, false);
}

// Both GEMMs of a small fp32 layer backward in one launch (c3_gemm_f32_bwd*):
// taken when each would run as a plain 64x64-tile launch (no split-K, no
// forced tile) and the two grids hold at most 128 tiles together, where a
// launch costs more than the k-loop it carries.  Same blocks, tile walks and arithmetic as the two
// separate launches.  C3HIP_ERR_UNSUPPORTED: not applicable, nothing launched.
int linear_bwd_pair(const GemmArgs& ax, const GemmArgs& aw, bool relu, hipStream_t stream) {
    const Kind kx = relu ? Kind::DxMask : Kind::Dx, kw = relu ? Kind::DwMask : Kind::Dw;
    const Tile* t = &kF32Tiles[0];
    if (f32_forced() || choose_f32_tile(kx, ax.M, ax.N) != t || choose_f32_tile(kw, aw.M, aw.N) != t ||
        plan_split_f32(ax, t) || plan_split_f32(aw, t))
        return C3HIP_ERR_UNSUPPORTED;
    const int64_t nx = tile_count(ax, t), nw = tile_count(aw, t);
    if (nx + nw > 128) return C3HIP_ERR_UNSUPPORTED;
    const bool vec = vec_ok(true, ax.M, ax.K, ax.lda, ax.A, ax.Amask) && vec_ok(true, ax.N, ax.K, ax.ldb, ax.B, ax.Bmask) &&
                     vec_ok(false, aw.M, aw.K, aw.lda, aw.A, aw.Amask) && vec_ok(false, aw.N, aw.K, aw.ldb, aw.B, aw.Bmask);
    BwdPairArgs p{};
    p.dx = ax;
    p.dw = aw;
    p.nx = (int)nx;
    char name[64];
    std::snprintf(name, sizeof(name), "c3_gemm_f32_bwd%s_%s_%s", relu ? "_mask" : "",
                  ax.K <= 128 && aw.K <= 128 && vec ? "t64x64k" : "t64x64", vec ? "v" : "s");
    void* args[] = {&p};
    return launch(name, dim3((unsigned)(nx + nw)), dim3(t->threads), args, stream);
}

int c3hip_linear_bwd(int dtype, const void* X, const void* W, const void* Y, const void* dY, void* dX, float* dW,
                     float* db, int64_t M, int64_t K, int64_t N, int act, void* stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    int rc = check_dtype(dtype);
    if (rc) return rc;
    if (act < C3HIP_ACT_NONE || act > C3HIP_ACT_TANH) return set_error(C3HIP_ERR_INVALID, "unknown act");
    if ((rc = check_elems("X", M, K)) || (rc = check_elems("W", K, N)) || (rc = check_elems("dY", M, N))) return rc;
    const bool relu = act == C3HIP_ACT_RELU;
    if (M > 0 && N > 0 && (!dY || (act != C3HIP_ACT_NONE && !Y))) return set_error(C3HIP_ERR_INVALID, "null dY / Y");
    if (dX && K > 0 && M > 0 && N > 0 && !W) return set_error(C3HIP_ERR_INVALID, "dX needs W");
    if (dW && K > 0 && N > 0 && M > 0 && !X) return set_error(C3HIP_ERR_INVALID, "dW needs X");
    if (dtype == C3HIP_BF16 || act == C3HIP_ACT_SIGMOID || act == C3HIP_ACT_TANH)
        return linear_bwd_prepass(dtype, X, W, Y, dY, dX, dW, db, M, K, N, act, stream);
    const void* mask = relu ? Y : nullptr;
    // dX[M,K] = dZ[M,N] . W^T : logical (M, N=K, K=N), A = dY (k-contig), B(k=n, j) = W[j*N + n].
    GemmArgs ax{};
    ax.A = dY; ax.Amask = mask; ax.B = W; ax.C = dX;
    ax.M = M; ax.N = K; ax.K = N;
    ax.lda = N; ax.ldb = N; ax.ldc = K;
    // dW[K,N] = X^T . dZ : logical (M=K, N, K=M), A(i, m) = X[m*K + i], B(m, j) = dZ[m*N + j].
    GemmArgs aw{};
    aw.A = X; aw.B = dY; aw.Bmask = mask; aw.C = dW; aw.db = db;
    aw.M = K; aw.N = N; aw.K = M;
    aw.lda = K; aw.ldb = N; aw.ldc = N;
    if (dX && dW && M > 0 && N > 0 && K > 0) {
        rc = linear_bwd_pair(ax, aw, relu, stream);
        if (rc != C3HIP_ERR_UNSUPPORTED) return rc;  // launched (or failed); unsupported: separate launches
        clear_error();
    }
    if (relu && M > 0 && N > 0 && K > 0 && f32_bwd_direct(ax, aw, Y, dY))
        return linear_bwd_prepass(dtype, X, W, Y, dY, dX, dW, db, M, K, N, act, stream);
    if (relu && dX && dW && M > 0 && N > 0 && K > 0) {
        // Both GEMMs: dX forms dZ = mask(Y) * dY in its operand loads anyway,
        // so it also writes dZ (each k-tile once, from the staging registers)
        // and dW + db run on dZ as a plain GEMM, which reads 4 bytes per
        // element of the k = M operand instead of 8 (dY and Y).  The products
        // are the same IEEE operations, so every output has the bits of the
        // masked launches.  Without memory for dZ, the masked launches run.
        void* dz = nullptr;
        WsHow how;
        if (take_workspace(nullptr, (size_t)(M * N) * sizeof(float), stream, &dz, &how, "dZ") == C3HIP_OK) {
            GemmArgs a1 = ax;
            a1.dz = dz;
            rc = run_gemm(dtype, Kind::DxMaskDz, a1, true, true, stream);
            if (rc == C3HIP_OK) {
                GemmArgs a2 = aw;
                a2.B = dz;
                a2.Bmask = nullptr;
                rc = run_gemm(dtype, Kind::Dw, a2, false, false, stream);
            }
            return release_workspace(dz, how, rc, stream, "dZ");
        }
        clear_error();
    }
    if (dX) {
        rc = run_gemm(dtype, relu ? Kind::DxMask : Kind::Dx, ax, true, true, stream);
        if (rc) return rc;
    }
    if (dW) {
        GemmArgs& a = aw;
        if (K == 0 && db) {
            // No dW rows: no block would visit dY, so the column sums run on their own.
            a.db = nullptr;
        } else {
            rc = run_gemm(dtype, relu ? Kind::DwMask : Kind::Dw, a, false, false, stream);
            if (rc) return rc;
            if (N > 0 && a.db) return C3HIP_OK;
        }
    }
    if (db && (!dW || K == 0)) {
        if (dtype != C3HIP_F32) return set_error(C3HIP_ERR_UNSUPPORTED, "bf16 db without dW");
        return colsum((const float*)dY, (const float*)mask, db, M, N, stream);
    }
    return C3HIP_OK;
}

int c3hip_sum_reduce(const float* in, float* out, int64_t M, int64_t N, int axis, void* stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    if (axis != 0 && axis != 1) return set_error(C3HIP_ERR_INVALID, "axis must be 0 or 1");
    if (M < 0 || N < 0) return set_error(C3HIP_ERR_INVALID, "negative dimension");
    const int64_t outn = axis == 0 ? N : M;
    if (outn == 0) return C3HIP_OK;
    if (!out || (M > 0 && N > 0 && !in)) return set_error(C3HIP_ERR_INVALID, "null pointer");
    if (axis == 0) return colsum(in, nullptr, out, M, N, stream);
    void* args[] = {(void*)&in, (void*)&out, &M, &N};
    return launch("c3_rowsum_f32", dim3((unsigned)((M + 3) / 4)), dim3(256), args, stream);
}

}  // extern "C"
