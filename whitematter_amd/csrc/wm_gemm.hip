// wm_gemm.hip -- fp32 matrix products on the gfx950 matrix cores
// (include/wm_gemm.h): Tensor::matmul / bmm and their backward
// (core/tensor.cpp:783-895), and the strided product the drop-in Linear and
// MultiHeadAttention modules use.
//
// gemm_kernel covers every case (gemm_dma_kernel, below, takes a subset
// faster).  A workgroup of 4 waves computes a 128 x 128 tile of C; each wave a 64 x 64 quarter as 2 x 2 blocks of
// v_mfma_f32_32x32x2_f32.  k advances in stages of 32: the next stage's tiles
// of op(A) and op(B) are loaded from HBM into registers while the matrix
// cores work on the current ones from LDS (two LDS buffers, one barrier per
// stage).
//
// Each operand tile keeps its HBM orientation in LDS, so every global load
// is a float4 along the contiguous dimension and every LDS write is a plain
// vector store:
//   k-contiguous operands (A untransposed, B transposed): LDS [row][k] with a
//     36-float pitch; an MFMA fragment is four 16-byte LDS reads;
//   row-contiguous operands (A transposed, B untransposed): LDS [k][row]
//     with a 130-float pitch; a fragment is one 4-byte read per k.
// An MFMA step takes two k values per lane (one per half-wave).  Which k
// goes to which step is free as long as A and B agree: half h takes
// k = 16h .. 16h+15 of the stage.  The pitches keep a quarter-wave's reads
// on distinct banks, and the two half-waves' rows 16 k apart on opposite
// halves of the banks (16 * 130 = 32 mod 64).
//
// Interior tiles load and store without bounds checks; tiles on the edge of
// C or the last k stage take an element-wise path that reads only inside
// the operands and zero-fills the rest.
//
// A launch with fewer tiles than CUs and a long k (a weight gradient
// x^T dY: small m x n, k = every row of the batch) splits k into slices:
// each slice's product goes to a workspace and a second pass adds the slices
// in fixed order, scales and accumulates into C.
//
// Products whose tiles are all interior (m, n multiples of 128, k of 64,
// 16-byte rows; one batch level) take gemm_dma_kernel instead: the
// operands go from global memory straight into LDS (no registers held for
// them), in stages of 16 k over four LDS buffers with three stages in flight,
// and a workgroup runs the same tile of two consecutive problems, moving the
// second problem's first stages while the first one's C is written.  At
// k = 128 a tile's stages are too few for one stage of look-ahead to hide
// the loads, which bounds gemm_kernel there (see the kernel's comment).
//
// Sums are fp32 in the matrix cores' order (see include/wm_gemm.h).
#include "wm_common.hpp"

#include "../../include/wm_gemm.h"

#include <rocblas/rocblas.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <mutex>

namespace wm {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTile = 128;      // C tile rows per workgroup (columns: BN = 128 or 64)
constexpr int kBK = 32;         // k per stage
constexpr int kPitchK = kBK + 4;      // LDS [row][k] pitch (floats)
constexpr int kThreads = 256;   // 4 waves as 2 x 2, each 64 x BN/2 of C
// LDS [k][row] pitch for an operand tile of R rows: R + 2 keeps a
// quarter-wave's 4-byte reads on distinct banks and puts the two half-waves'
// rows (16 k apart) on opposite halves of the banks (16 (R + 2) = 32 mod 64).
template <int R>
constexpr int pitch_r() { return R + 2; }
constexpr int kOperandFloats = kTile * kPitchK > kBK * (kTile + 2) ? kTile * kPitchK : kBK * (kTile + 2);

struct GemmParams {
    const float* a;
    const float* b;
    float* c;
    const float* bias;
    int64_t m, n, k, lda, ldb, ldc;
    int64_t batch, batch_inner;
    int64_t sa0, sa1, sb0, sb1, sc0, sc1;
    float alpha;
    int accumulate;
    int tiles_m, tiles_n;
    int c_aligned;  // C and every problem's C start 16-byte aligned
    // Split k: each problem runs as kslices products over k slices of ksplit
    // (a multiple of kBK); slice s writes its own C at + s * sck.
    int kslices;
    int64_t ksplit, sck;
    int group;  // gemm_dma_kernel: consecutive problems per workgroup
};

// One operand's R x 32 tile per stage (R = 128 or 64 rows of op(A), or
// columns of op(B), by k).  KC: element (r, kk) at base[r * ld + kk], else
// at base[kk * ld + r].  Each thread moves NS = R / 32 float4s:
//   KC:  slot i = row t/8 + 32 i, k 4 (t % 8) .. + 3          -> LDS [row][k]
//   !KC: slot i = k t/L + (256/L) i, rows 4 (t % L) .. + 3,    -> LDS [k][row]
//        with L = R / 4 lanes across the rows
template <bool KC, int R>
struct Operand {
    static constexpr int NS = R / 32;
    static constexpr int L = R / 4;
    static constexpr int KSTEP = kThreads / L;  // k rows per slot (!KC)
    static constexpr int PR = pitch_r<R>();
    const float* base;
    int64_t ld, rows, r0;
    int64_t lane_off;  // this thread's first element relative to (r0, k0 = 0)
    float4 v[NS];

    __device__ __forceinline__ void init(const float* b, int64_t ld_, int64_t rows_, int64_t r0_) {
        const int t = (int)threadIdx.x;
        base = b;
        ld = ld_;
        rows = rows_;
        r0 = r0_;
        lane_off = KC ? (r0 + t / 8) * ld + 4 * (t % 8) : (int64_t)(t / L) * ld + r0 + 4 * (t % L);
    }

    // Interior tile, whole stage inside k, 16-byte aligned rows.
    __device__ __forceinline__ void load_fast(int64_t k0) {
        const float* p = base + lane_off + (KC ? k0 : k0 * ld);
        const int64_t step = KC ? 32 * ld : KSTEP * ld;
#pragma unroll
        for (int i = 0; i < NS; ++i) v[i] = *reinterpret_cast<const float4*>(p + i * step);
    }

    // Any tile: element by element, reading only inside rows x kdim.
    __device__ __forceinline__ void load_edge(int64_t kdim, int64_t k0) {
        const int t = (int)threadIdx.x;
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            float e[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t r = KC ? r0 + t / 8 + 32 * i : r0 + 4 * (t % L) + j;
                const int64_t kk = KC ? k0 + 4 * (t % 8) + j : k0 + t / L + KSTEP * i;
                e[j] = (r < rows && kk < kdim) ? (KC ? base[r * ld + kk] : base[kk * ld + r]) : 0.0f;
            }
            v[i] = make_float4(e[0], e[1], e[2], e[3]);
        }
    }

    __device__ __forceinline__ void store(float* lds) const {
        const int t = (int)threadIdx.x;
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if constexpr (KC) {
                *reinterpret_cast<float4*>(lds + (t / 8 + 32 * i) * kPitchK + 4 * (t % 8)) = v[i];
            } else {
                float* q = lds + (t / L + KSTEP * i) * PR + 4 * (t % L);
                *reinterpret_cast<float2*>(q) = make_float2(v[i].x, v[i].y);
                *reinterpret_cast<float2*>(q + 2) = make_float2(v[i].z, v[i].w);
            }
        }
    }

    // Fragment values of tile row `row`, k = kk .. kk + 3 of the stage.
    __device__ __forceinline__ static float4 frag(const float* lds, int row, int kk) {
        if constexpr (KC) {
            return *reinterpret_cast<const float4*>(lds + row * kPitchK + kk);
        } else {
            return make_float4(lds[kk * PR + row], lds[(kk + 1) * PR + row], lds[(kk + 2) * PR + row],
                               lds[(kk + 3) * PR + row]);
        }
    }
};

// Tile order inside one problem: groups of 8 tile-rows walked column by
// column, so the workgroups resident at one time share panels of A and B.
__device__ __forceinline__ void tile_of(int t, int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int kGroup = 8;
    const int per_group = kGroup * tiles_n;
    const int g = t / per_group;
    const int first = g * kGroup;
    const int rows = min(tiles_m - first, kGroup);
    const int in = t - g * per_group;
    tm = first + in % rows;
    tn = in / rows;
}

template <bool TA, bool TB, bool VEC, int BN>
__global__ void __launch_bounds__(kThreads) gemm_kernel(GemmParams P) {
    constexpr int JB = BN / 64;  // 32-column blocks per wave (each wave: 64 x BN/2)
    __shared__ __attribute__((aligned(16))) float lds[2][2][kOperandFloats];  // [stage][A, B]

    const int ntiles = P.tiles_m * P.tiles_n;
    // Workgroups are dealt to the 8 XCDs in turn; renumber them so each XCD
    // (own L2) takes a contiguous run of tiles.
    int t = (int)blockIdx.x;
    if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
    int tm, tn;
    tile_of(t, P.tiles_m, P.tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * BN;
    const bool interior = VEC && m0 + kTile <= P.m && n0 + BN <= P.n;

    const int lane = (int)threadIdx.x & 63;
    const int wave = (int)threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, r = lane & 31;

    // op(A) row r, k kk: A[r * lda + kk] (TA = 0) or A[kk * lda + r].
    // op(B) column r, k kk: B[kk * ldb + r] (TB = 0) or B[r * ldb + kk].
    using OpA = Operand<!TA, kTile>;
    using OpB = Operand<TB, BN>;

    const int64_t nprob = P.batch * P.kslices;
    for (int64_t p = blockIdx.y; p < nprob; p += gridDim.y) {
        const int64_t pb = p / P.kslices, ks = p - pb * P.kslices;
        const int64_t po = pb / P.batch_inner, pi = pb - po * P.batch_inner;
        const int64_t kb = ks * P.ksplit;  // first k of this slice
        const int64_t kdim = min(P.ksplit, P.k - kb);
        const int nk = (int)((kdim + kBK - 1) / kBK);
        const int nk_fast = interior ? (int)(kdim / kBK) : 0;  // stages that take the unchecked loads
        OpA a;
        OpB b;
        a.init(P.a + po * P.sa0 + pi * P.sa1 + (TA ? kb * P.lda : kb), P.lda, P.m, m0);
        b.init(P.b + po * P.sb0 + pi * P.sb1 + (TB ? kb : kb * P.ldb), P.ldb, P.n, n0);
        float* C = P.c + po * P.sc0 + pi * P.sc1 + ks * P.sck;
        const bool aligned_c = P.c_aligned != 0;

        f32x16 acc[2][JB];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < JB; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

        if (nk > 0) {
            if (nk_fast > 0) {
                a.load_fast(0);
                b.load_fast(0);
            } else {
                a.load_edge(kdim, 0);
                b.load_edge(kdim, 0);
            }
            a.store(lds[0][0]);
            b.store(lds[0][1]);
        }
        __syncthreads();

        for (int s = 0; s < nk; ++s) {
            const int cur = s & 1;
            const bool more = s + 1 < nk;
            if (more) {
                const int64_t k0 = (int64_t)(s + 1) * kBK;
                if (s + 1 < nk_fast) {
                    a.load_fast(k0);
                    b.load_fast(k0);
                } else {
                    a.load_edge(kdim, k0);
                    b.load_edge(kdim, k0);
                }
            }
            const float* As = lds[cur][0];
            const float* Bs = lds[cur][1];
#pragma unroll
            for (int kq = 0; kq < 4; ++kq) {
                const int kk = 16 * half + 4 * kq;
                float4 av[2], bv[JB];
#pragma unroll
                for (int i = 0; i < 2; ++i) av[i] = OpA::frag(As, wm * 64 + i * 32 + r, kk);
#pragma unroll
                for (int j = 0; j < JB; ++j) bv[j] = OpB::frag(Bs, wn * (BN / 2) + j * 32 + r, kk);
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < JB; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].x, bv[j].x, acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].y, bv[j].y, acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].z, bv[j].z, acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].w, bv[j].w, acc[i][j], 0, 0, 0);
                    }
            }
            if (more) {
                a.store(lds[cur ^ 1][0]);
                b.store(lds[cur ^ 1][1]);
            }
            __syncthreads();
        }

        // Epilogue through LDS: each wave parks its 64 x BN/2 quarter (4 floats
        // of row padding) in its own slice of the stage buffers, which the
        // last barrier freed, then writes C as float4 rows: LPR lanes per row
        // of the quarter, RPP rows per pass.
        // Accumulator element q of a 32 x 32 block sits at row
        // 8 * (q / 4) + 4 * half + q % 4, column r.
        constexpr int kEp = BN / 2 + 4;
        constexpr int LPR = BN / 8, RPP = 64 / LPR;
        float* ep = &lds[0][0][0] + wave * 64 * kEp;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < JB; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    ep[(i * 32 + 8 * (q >> 2) + 4 * half + (q & 3)) * kEp + j * 32 + r] = acc[i][j][q];
        const float alpha = P.alpha;
        const bool accum = P.accumulate != 0;
        const int cq = (lane % LPR) * 4;  // this lane's 4 columns within the quarter
        const int64_t col = n0 + wn * (BN / 2) + cq;
        const bool vec_c = interior && (P.ldc & 3) == 0 && aligned_c;
        float4 bias4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (P.bias) {
            float bb[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) bb[e] = (interior || col + e < P.n) ? P.bias[col + e] : 0.0f;
            bias4 = make_float4(bb[0], bb[1], bb[2], bb[3]);
        }
#pragma unroll 4
        for (int s4 = 0; s4 < 64 / RPP; ++s4) {
            const int rq = lane / LPR + RPP * s4;  // row within the quarter
            const int64_t row = m0 + wm * 64 + rq;
            const float4 a4 = *reinterpret_cast<const float4*>(ep + rq * kEp + cq);
            float4 v = make_float4(alpha * a4.x, alpha * a4.y, alpha * a4.z, alpha * a4.w);
            float* dst = C + row * P.ldc + col;
            if (vec_c) {
                if (accum) {
                    const float4 old = *reinterpret_cast<const float4*>(dst);
                    v = make_float4(old.x + v.x, old.y + v.y, old.z + v.z, old.w + v.w);
                }
                if (P.bias) v = make_float4(v.x + bias4.x, v.y + bias4.y, v.z + bias4.z, v.w + bias4.w);
                // C is written once: streaming stores keep it from evicting
                // the A and B panels that the resident tiles re-read from the
                // caches (bmm at k = 128: 0.188 -> 0.181 ms).
                if (accum) *reinterpret_cast<float4*>(dst) = v;
                else st_stream(dst, v);
            } else if (row < P.m) {
                const float ve[4] = {v.x, v.y, v.z, v.w}, be[4] = {bias4.x, bias4.y, bias4.z, bias4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (col + e >= P.n) continue;
                    float x = ve[e];
                    if (accum) x = dst[e] + x;
                    if (P.bias) x = x + be[e];
                    dst[e] = x;
                }
            }
        }
        __syncthreads();  // the next problem's first stage reuses LDS buffer 0
    }
}

// ---- interior products: operands straight into LDS -----------------------
//
// gemm_dma_kernel computes the same 128 x 128 C tiles as gemm_kernel, with the
// same waves, MFMA blocks and LDS-staged epilogue, for products whose tiles
// are all interior (checked on the host).  What changes is how the operands
// reach LDS:
//   - global_load_lds_dwordx4 moves 16 bytes per lane from global memory to
//     LDS at M0 + 16 * lane, so no registers hold the next stages;
//   - k advances in stages of 16 over four LDS buffers with three stages in
//     flight (48 k ahead of the matrix cores), where one stage of 32 in
//     registers could not hide the loads behind a small-k tile's few stages;
//   - a workgroup takes the same tile of `group` consecutive problems, and
//     starts the next problem's first two stages as soon as the last stage's
//     barrier frees the buffers, while the epilogue writes C through the
//     other two.
// Per stage each wave moves two 1 KB blocks of each operand (block
// i = 2 wave + u), by the operand's layout in memory (DmaOperand):
//   k-contiguous (A untransposed, B transposed): tile rows 16 i .. 16 i + 15
//     at 64 bytes each; lane l fills row 16 i + l / 4, 16-byte slot l % 4,
//     with k chunk slot ^ swz(row), swz(row) = ((row >> 1) ^ (row >> 2)) & 3,
//     so the fragment reads (one row per lane, one chunk) fall on distinct
//     banks for 32 and for 64 banks of LDS;
//   row-contiguous (A transposed, B untransposed): k rows 2 i and 2 i + 1 at
//     512 bytes each; lane l fills k row 2 i + l / 32, tile rows
//     4 (l % 32) .. + 3.
// Half-wave h takes k = 8 h .. 8 h + 7 of a stage (chunks 2 h and 2 h + 1).
//
// The transfers are issued from inline asm: the compiler cannot tell which
// buffer a transfer writes, and for builtin transfers it waits for all of
// them before every LDS read.  The kernel orders them itself: before stage s
// each wave waits until at most as many vector memory operations are in
// flight as it issued transfers after stage s's (those of stages s + 1 and
// s + 2), then a barrier makes every wave's transfers visible; a buffer is
// refilled only after the barrier that follows its last reads.  Transfers
// are loads and complete in issue order; C's stores from the previous
// problem, counted by the same counter, can only make such a wait stricter.
// An opaque transfer can only make the compiler's own waits stricter too.
constexpr int kDK = 16;                              // k per stage
constexpr int kDStageFloats = 2 * kTile * kDK;       // A [128][16] + B [16][128]
constexpr int kDEp = 64 + 4;                         // epilogue row pitch (floats)
constexpr int kDBufFloats = kDStageFloats > 64 * kDEp ? kDStageFloats : 64 * kDEp;

__device__ __forceinline__ void lgkm_wait0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Wait until at most `outstanding` (0, 4 or 8) vector memory operations of
// this wave are in flight.
__device__ __forceinline__ void vm_wait_upto(int outstanding) {
    if (outstanding >= 8) __builtin_amdgcn_s_waitcnt(0x0F78);
    else if (outstanding >= 4) __builtin_amdgcn_s_waitcnt(0x0F74);
    else __builtin_amdgcn_s_waitcnt(0x0F70);
}

// 16 bytes per lane from g to LDS byte address lds + 16 * lane (lds
// wave-uniform, in M0).  M0 is declared clobbered; the compiler warns that
// it reserves M0, and gemm_dma_kernel's code has no other use of it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const float* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// s_barrier with the compiler kept from moving memory accesses across it.
__device__ __forceinline__ void wg_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One operand's staging in gemm_dma_kernel.  KC: element (row, k) at
// base[row * ld + k] (A untransposed, B transposed), staged as rows of 16 k
// in swizzled 16-byte chunks; else at base[k * ld + row] (A transposed, B
// untransposed), staged as k rows of 128.
template <bool KC>
struct DmaOperand {
    // This lane's source for transfer u (block i = 2 wave + u) at k = 0.
    __device__ __forceinline__ static int64_t src(int64_t ld, int64_t r0, int wave, int lane, int u) {
        const int i = 2 * wave + u;
        if constexpr (KC) {
            const int row = 16 * i + lane / 4;
            return (r0 + row) * ld + 4 * ((lane & 3) ^ (((row >> 1) ^ (row >> 2)) & 3));
        } else {
            return (int64_t)(2 * i + lane / 32) * ld + r0 + 4 * (lane & 31);
        }
    }
    __device__ __forceinline__ static int64_t k_step(int64_t k0, int64_t ld) { return KC ? k0 : k0 * ld; }
    // Fragment of tile row R: k = 8 half + 4 kq .. + 3 of the stage.
    __device__ __forceinline__ static float4 frag(const float* T, int R, int half, int kq) {
        if constexpr (KC) {
            const int c = 2 * half + kq;
            return *reinterpret_cast<const float4*>(T + R * kDK + 4 * (c ^ (((R >> 1) ^ (R >> 2)) & 3)));
        } else {
            const int kr = 8 * half + 4 * kq;
            return make_float4(T[kr * kTile + R], T[(kr + 1) * kTile + R], T[(kr + 2) * kTile + R],
                               T[(kr + 3) * kTile + R]);
        }
    }
};

template <bool TA, bool TB>
__global__ void __launch_bounds__(kThreads) gemm_dma_kernel(GemmParams P) {
    using OpA = DmaOperand<!TA>;
    using OpB = DmaOperand<TB>;
    // Four stage buffers; each also holds one wave's half epilogue quarter.
    __shared__ __attribute__((aligned(16))) float lds0[kDBufFloats];
    __shared__ __attribute__((aligned(16))) float lds1[kDBufFloats];
    __shared__ __attribute__((aligned(16))) float lds2[kDBufFloats];
    __shared__ __attribute__((aligned(16))) float lds3[kDBufFloats];
    auto bufp = [&](int bi) -> float* { return bi == 0 ? lds0 : bi == 1 ? lds1 : bi == 2 ? lds2 : lds3; };
    auto lds_addr = [&](int bi) -> uint32_t {
        return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)bufp(bi);
    };

    const int ntiles = P.tiles_m * P.tiles_n;
    int t = (int)blockIdx.x;
    if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
    int tm, tn;
    tile_of(t, P.tiles_m, P.tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
    const int lane = (int)threadIdx.x & 63;
    const int wave = (int)threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, r = lane & 31;

    int64_t aoff[2], boff[2];  // this lane's sources at k = 0
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        aoff[u] = OpA::src(P.lda, m0, wave, lane, u);
        boff[u] = OpB::src(P.ldb, n0, wave, lane, u);
    }
    const int nk = (int)(P.k / kDK);
    const uint32_t wofs = (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 2048u;  // the wave's two blocks
    auto issue = [&](int64_t pp, int st, int bi) {  // stage st of problem pp into buffer bi
        const float* Ab = P.a + pp * P.sa0;
        const float* Bb = P.b + pp * P.sb0;
        const int64_t k0 = (int64_t)st * kDK;
        const uint32_t la = lds_addr(bi) + wofs;
#pragma unroll
        for (int u = 0; u < 2; ++u) lds_dma16(Ab + aoff[u] + OpA::k_step(k0, P.lda), la + 1024u * u);
#pragma unroll
        for (int u = 0; u < 2; ++u)
            lds_dma16(Bb + boff[u] + OpB::k_step(k0, P.ldb), la + 4u * kTile * kDK + 1024u * u);
    };

    int64_t p = (int64_t)blockIdx.y * P.group;
    const int64_t pend = min(P.batch, p + (int64_t)P.group);
    issue(p, 0, 0);
    issue(p, 1, 1);
    issue(p, 2, 2);
    for (; p < pend; ++p) {
        float* C = P.c + p * P.sc0;
        f32x16 acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
        // nk is a multiple of 4: unrolled over the buffers, so every LDS
        // address below is a constant offset.
        for (int s0 = 0; s0 < nk; s0 += 4) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int s = s0 + b;
                vm_wait_upto(4 * min(nk - 1 - s, 2));
                lgkm_wait0();
                wg_barrier();
                if (s + 3 < nk) issue(p, s + 3, (b + 3) & 3);
                const float* As = bufp(b);
                const float* Bs = As + kTile * kDK;
#pragma unroll
                for (int kq = 0; kq < 2; ++kq) {
                    float4 av[2], bv[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) av[i] = OpA::frag(As, wm * 64 + i * 32 + r, half, kq);
#pragma unroll
                    for (int j = 0; j < 2; ++j) bv[j] = OpB::frag(Bs, wn * 64 + j * 32 + r, half, kq);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].x, bv[j].x, acc[i][j], 0, 0, 0);
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].y, bv[j].y, acc[i][j], 0, 0, 0);
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].z, bv[j].z, acc[i][j], 0, 0, 0);
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].w, bv[j].w, acc[i][j], 0, 0, 0);
                        }
                }
            }
        }
        lgkm_wait0();
        wg_barrier();  // every wave is done with the stage buffers
        const bool more = p + 1 < pend;
        if (more) {
            issue(p + 1, 0, 0);
            issue(p + 1, 1, 1);
        }
        // Epilogue through buffers 2 and 3: each wave parks half of its
        // 64 x 64 quarter at a time (accumulator element q of a 32 x 32 block
        // at row 8 (q / 4) + 4 half + q % 4, column r), then writes it as
        // float4 rows, 16 lanes per 256-byte row segment.
        float* ep = bufp(2 + (wave >> 1)) + (wave & 1) * 32 * kDEp;
        const float alpha = P.alpha;
        const bool accum = P.accumulate != 0;
        const int cq = (lane % 16) * 4;
        const int64_t col = n0 + wn * 64 + cq;
        float4 bias4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (P.bias) bias4 = *reinterpret_cast<const float4*>(P.bias + col);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (i) lgkm_wait0();  // this wave's reads of the first half are done
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    ep[(8 * (q >> 2) + 4 * half + (q & 3)) * kDEp + j * 32 + r] = acc[i][j][q];
#pragma unroll 4
            for (int s4 = 0; s4 < 8; ++s4) {
                const int rq = lane / 16 + 4 * s4;
                const int64_t row = m0 + wm * 64 + i * 32 + rq;
                const float4 a4 = *reinterpret_cast<const float4*>(ep + rq * kDEp + cq);
                float4 v = make_float4(alpha * a4.x, alpha * a4.y, alpha * a4.z, alpha * a4.w);
                float* dst = C + row * P.ldc + col;
                if (accum) {
                    const float4 old = *reinterpret_cast<const float4*>(dst);
                    v = make_float4(old.x + v.x, old.y + v.y, old.z + v.z, old.w + v.w);
                }
                if (P.bias) v = make_float4(v.x + bias4.x, v.y + bias4.y, v.z + bias4.z, v.w + bias4.w);
                if (accum) *reinterpret_cast<float4*>(dst) = v;
                else st_stream(dst, v);
            }
        }
        lgkm_wait0();
        wg_barrier();  // every wave is done with buffers 2 and 3
        if (more) issue(p + 1, 2, 2);
    }
}

// gemm_dma3_kernel is gemm_dma_kernel with three stage buffers of 16 k (two
// stages in flight) and a 52 KB LDS footprint, so three workgroups share a
// CU instead of two; the epilogue goes through the third buffer in four
// 16-row slices of each wave's quarter.  It is launched for k <= 256, where
// a tile's few stages leave most of its time in set-up and epilogue, which a
// third co-resident tile covers: bmm [64, 1024, 128] forward 67.1 -> 71.5 %
// of the matrix peak (means of four runs on one box).  At k = 1024 two
// stages of look-ahead are too few (74.3 -> 69.7 %), so longer products keep
// gemm_dma_kernel.  The buffer index is a runtime value (the transfers are
// opaque to the compiler).
constexpr int kD3Buf = kDStageFloats > 4 * 16 * kDEp ? kDStageFloats : 4 * 16 * kDEp;  // a stage or a 16-row slice of all 4 quarters

template <bool TA, bool TB>
__global__ void __launch_bounds__(kThreads) gemm_dma3_kernel(GemmParams P) {
    using OpA = DmaOperand<!TA>;
    using OpB = DmaOperand<TB>;
    __shared__ __attribute__((aligned(16))) float lds[3 * kD3Buf];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)lds;

    const int ntiles = P.tiles_m * P.tiles_n;
    int t = (int)blockIdx.x;
    if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
    int tm, tn;
    tile_of(t, P.tiles_m, P.tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
    const int lane = (int)threadIdx.x & 63;
    const int wave = (int)threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, r = lane & 31;

    int64_t aoff[2], boff[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        aoff[u] = OpA::src(P.lda, m0, wave, lane, u);
        boff[u] = OpB::src(P.ldb, n0, wave, lane, u);
    }
    const int nk = (int)(P.k / kDK);
    const uint32_t wofs = (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 2048u;
    auto issue = [&](int64_t pp, int st, int bi) {
        const float* Ab = P.a + pp * P.sa0;
        const float* Bb = P.b + pp * P.sb0;
        const int64_t k0 = (int64_t)st * kDK;
        const uint32_t la = lds0 + 4u * (uint32_t)(bi * kD3Buf) + wofs;
#pragma unroll
        for (int u = 0; u < 2; ++u) lds_dma16(Ab + aoff[u] + OpA::k_step(k0, P.lda), la + 1024u * u);
#pragma unroll
        for (int u = 0; u < 2; ++u)
            lds_dma16(Bb + boff[u] + OpB::k_step(k0, P.ldb), la + 4u * kTile * kDK + 1024u * u);
    };

    int64_t p = (int64_t)blockIdx.y * P.group;
    const int64_t pend = min(P.batch, p + (int64_t)P.group);
    issue(p, 0, 0);
    issue(p, 1, 1);
    for (; p < pend; ++p) {
        float* C = P.c + p * P.sc0;
        f32x16 acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
        for (int s = 0; s < nk; ++s) {
            // at most stage s + 1's transfers in flight (see gemm_dma_kernel)
            if (s + 1 < nk) __builtin_amdgcn_s_waitcnt(0x0F74);
            else __builtin_amdgcn_s_waitcnt(0x0F70);
            lgkm_wait0();
            wg_barrier();
            if (s + 2 < nk) issue(p, s + 2, (s + 2) % 3);
            const float* As = lds + (s % 3) * kD3Buf;
            const float* Bs = As + kTile * kDK;
#pragma unroll
            for (int kq = 0; kq < 2; ++kq) {
                float4 av[2], bv[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) av[i] = OpA::frag(As, wm * 64 + i * 32 + r, half, kq);
#pragma unroll
                for (int j = 0; j < 2; ++j) bv[j] = OpB::frag(Bs, wn * 64 + j * 32 + r, half, kq);
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].x, bv[j].x, acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].y, bv[j].y, acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].z, bv[j].z, acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].w, bv[j].w, acc[i][j], 0, 0, 0);
                    }
            }
        }
        lgkm_wait0();
        wg_barrier();  // every wave is done with the stage buffers
        const bool more = p + 1 < pend;
        if (more) {
            issue(p + 1, 0, 0);
            issue(p + 1, 1, 1);
        }
        // Epilogue through buffer 2 (0 and 1 may be filling) in four 16-row
        // slices of each wave's quarter.
        float* ep = lds + 2 * kD3Buf + wave * 16 * kDEp;
        const float alpha = P.alpha;
        const bool accum = P.accumulate != 0;
        const int cq = (lane % 16) * 4;
        const int64_t col = n0 + wn * 64 + cq;
        float4 bias4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (P.bias) bias4 = *reinterpret_cast<const float4*>(P.bias + col);
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) {
            const int i = sl >> 1, e0 = 8 * (sl & 1);
            if (sl) lgkm_wait0();  // this wave's reads of the previous slice are done
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int q = e0 + e;
                    ep[(8 * ((q >> 2) - 2 * (sl & 1)) + 4 * half + (q & 3)) * kDEp + j * 32 + r] = acc[i][j][q];
                }
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int rq = lane / 16 + 4 * s4;
                const int64_t row = m0 + wm * 64 + 16 * sl + rq;
                const float4 a4 = *reinterpret_cast<const float4*>(ep + rq * kDEp + cq);
                float4 v = make_float4(alpha * a4.x, alpha * a4.y, alpha * a4.z, alpha * a4.w);
                float* dst = C + row * P.ldc + col;
                if (accum) {
                    const float4 old = *reinterpret_cast<const float4*>(dst);
                    v = make_float4(old.x + v.x, old.y + v.y, old.z + v.z, old.w + v.w);
                }
                if (P.bias) v = make_float4(v.x + bias4.x, v.y + bias4.y, v.z + bias4.z, v.w + bias4.w);
                if (accum) *reinterpret_cast<float4*>(dst) = v;
                else st_stream(dst, v);
            }
        }
        lgkm_wait0();
        wg_barrier();  // every wave is done with buffer 2
    }
}

// ---- narrow interior products (n = 64): 32-k stages straight into LDS ----
//
// gemm_dma32_kernel is gemm_dma_kernel's staging for 128 x 64 C tiles (the
// attention's per-head products with 64-wide heads, two-level batches
// included): with 64-wide tiles a 16-k stage gives each wave too little
// matrix work against its waits and barrier, so k advances in stages of 32
// over three LDS buffers (24 KB each), two stages in flight.  Each wave
// computes a 64 x 32 quarter as 2 blocks of v_mfma_f32_32x32x2_f32 and moves
// per stage four 1 KB blocks of op(A) and two of op(B):
//   k-contiguous operand: rows of 32 k (128 bytes), 8 rows per block; lane l
//     fills row 8 i + l / 8, 16-byte slot l % 8, with k chunk
//     slot ^ swz8(row), swz8(row) = (row ^ (row >> 3)) & 7, which keeps the
//     fragment reads on distinct banks for 32 and for 64 banks;
//   row-contiguous operand: k rows of R floats, 256 / R of them per block.
// Half-wave h takes k = 16 h .. 16 h + 15 of a stage (chunks 4 h .. 4 h + 3).
// Transfers, waits and barriers as in gemm_dma_kernel; the buffer index is a
// runtime value here (the transfers are opaque to the compiler, so nothing
// needs its offsets to be constants).  Launched for products with a
// transposed A only (the attention backward's dV = attn^T dctx and
// dK = ds^T Q: 160.5 -> 146.7 us each against gemm_kernel); with A
// untransposed (attn V, ds K) it measured slower than gemm_kernel's 64-wide
// tiles (164.5 -> 178.0 us).
constexpr int kNK = 32;                                // k per stage
constexpr int kNStageFloats = kTile * kNK + kNK * 64;  // A [128][32] + B [32][64]
constexpr int kNEp = 32 + 4;                           // epilogue row pitch (floats)

__device__ __forceinline__ int swz8(int row) { return (row ^ (row >> 3)) & 7; }

template <bool KC, int R>
struct Dma32Operand {
    static constexpr int NBLK = R * kNK * 4 / 1024 / 4;  // 1 KB blocks per wave per stage
    static constexpr int KPB = 256 / R;                  // row-contiguous: k rows per block
    static constexpr int LPK = R / 4;                    // row-contiguous: lanes per k row
    __device__ __forceinline__ static int64_t src(int64_t ld, int64_t r0, int wave, int lane, int u) {
        const int i = NBLK * wave + u;
        if constexpr (KC) {
            const int row = 8 * i + lane / 8;
            return (r0 + row) * ld + 4 * ((lane & 7) ^ swz8(row));
        } else {
            return (int64_t)(KPB * i + lane / LPK) * ld + r0 + 4 * (lane % LPK);
        }
    }
    __device__ __forceinline__ static int64_t k_step(int64_t k0, int64_t ld) { return KC ? k0 : k0 * ld; }
    // Fragment of tile row `row`: k = 16 half + 4 kq .. + 3 of the stage.
    __device__ __forceinline__ static float4 frag(const float* T, int row, int half, int kq) {
        if constexpr (KC) {
            const int c = 4 * half + kq;
            return *reinterpret_cast<const float4*>(T + row * kNK + 4 * (c ^ swz8(row)));
        } else {
            const int kr = 16 * half + 4 * kq;
            return make_float4(T[kr * R + row], T[(kr + 1) * R + row], T[(kr + 2) * R + row], T[(kr + 3) * R + row]);
        }
    }
};

template <bool TA, bool TB>
__global__ void __launch_bounds__(kThreads) gemm_dma32_kernel(GemmParams P) {
    using OpA = Dma32Operand<!TA, kTile>;
    using OpB = Dma32Operand<TB, 64>;
    constexpr int XFER = OpA::NBLK + OpB::NBLK;  // transfers per wave per stage
    __shared__ __attribute__((aligned(16))) float lds[3 * kNStageFloats];

    const int ntiles = P.tiles_m * P.tiles_n;
    int t = (int)blockIdx.x;
    if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
    int tm, tn;
    tile_of(t, P.tiles_m, P.tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * 64;
    const int lane = (int)threadIdx.x & 63;
    const int wave = (int)threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, r = lane & 31;

    int64_t aoff[OpA::NBLK], boff[OpB::NBLK];  // this lane's sources at k = 0
#pragma unroll
    for (int u = 0; u < OpA::NBLK; ++u) aoff[u] = OpA::src(P.lda, m0, wave, lane, u);
#pragma unroll
    for (int u = 0; u < OpB::NBLK; ++u) boff[u] = OpB::src(P.ldb, n0, wave, lane, u);
    const int nk = (int)(P.k / kNK);
    const uint32_t wv = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)lds;
    // Operand and output starts of problem pp = (o, i): o = pp / batch_inner.
    struct Bases {
        const float* a;
        const float* b;
        float* c;
    };
    auto bases = [&](int64_t pp) -> Bases {
        int64_t po = pp, pi = 0;
        if (P.batch_inner != 1) {
            po = (int64_t)((uint32_t)pp / (uint32_t)P.batch_inner);  // batch <= INT_MAX (host)
            pi = pp - po * P.batch_inner;
        }
        return {P.a + po * P.sa0 + pi * P.sa1, P.b + po * P.sb0 + pi * P.sb1, P.c + po * P.sc0 + pi * P.sc1};
    };
    auto issue = [&](const Bases& q, int st, int bi) {  // stage st into buffer bi
        const int64_t k0 = (int64_t)st * kNK;
        const uint32_t la = lds0 + 4u * (uint32_t)(bi * kNStageFloats);
#pragma unroll
        for (int u = 0; u < OpA::NBLK; ++u)
            lds_dma16(q.a + aoff[u] + OpA::k_step(k0, P.lda), la + 1024u * (OpA::NBLK * wv + u));
#pragma unroll
        for (int u = 0; u < OpB::NBLK; ++u)
            lds_dma16(q.b + boff[u] + OpB::k_step(k0, P.ldb), la + 4u * kTile * kNK + 1024u * (OpB::NBLK * wv + u));
    };

    int64_t p = (int64_t)blockIdx.y * P.group;
    const int64_t pend = min(P.batch, p + (int64_t)P.group);
    Bases cur = bases(p);
    issue(cur, 0, 0);
    if (nk > 1) issue(cur, 1, 1);
    for (; p < pend; ++p) {
        f32x16 acc[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][q] = 0.0f;
        for (int s = 0; s < nk; ++s) {
            // at most stage s + 1's transfers in flight (see gemm_dma_kernel)
            if (s + 1 < nk) __builtin_amdgcn_s_waitcnt(0x0F70 | XFER);
            else __builtin_amdgcn_s_waitcnt(0x0F70);
            lgkm_wait0();
            wg_barrier();
            if (s + 2 < nk) issue(cur, s + 2, (s + 2) % 3);
            const float* As = lds + (s % 3) * kNStageFloats;
            const float* Bs = As + kTile * kNK;
#pragma unroll
            for (int kq = 0; kq < 4; ++kq) {
                float4 av[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) av[i] = OpA::frag(As, wm * 64 + i * 32 + r, half, kq);
                const float4 bv = OpB::frag(Bs, wn * 32 + r, half, kq);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].x, bv.x, acc[i], 0, 0, 0);
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].y, bv.y, acc[i], 0, 0, 0);
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].z, bv.z, acc[i], 0, 0, 0);
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].w, bv.w, acc[i], 0, 0, 0);
                }
            }
        }
        lgkm_wait0();
        wg_barrier();  // every wave is done with the stage buffers
        float* C = cur.c;
        const bool more = p + 1 < pend;
        if (more) {
            cur = bases(p + 1);
            issue(cur, 0, 0);
            if (nk > 1) issue(cur, 1, 1);
        }
        // Epilogue through buffer 2: each wave parks half of its 64 x 32
        // quarter at a time, then writes it as float4 rows, 8 lanes per
        // 128-byte row segment.
        float* ep = lds + 2 * kNStageFloats + wave * 32 * kNEp;
        const float alpha = P.alpha;
        const bool accum = P.accumulate != 0;
        const int cq = (lane % 8) * 4;
        const int64_t col = n0 + wn * 32 + cq;
        float4 bias4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (P.bias) bias4 = *reinterpret_cast<const float4*>(P.bias + col);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (i) lgkm_wait0();  // this wave's reads of the first half are done
#pragma unroll
            for (int q = 0; q < 16; ++q) ep[(8 * (q >> 2) + 4 * half + (q & 3)) * kNEp + r] = acc[i][q];
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int rq = lane / 8 + 8 * s4;
                const int64_t row = m0 + wm * 64 + i * 32 + rq;
                const float4 a4 = *reinterpret_cast<const float4*>(ep + rq * kNEp + cq);
                float4 v = make_float4(alpha * a4.x, alpha * a4.y, alpha * a4.z, alpha * a4.w);
                float* dst = C + row * P.ldc + col;
                if (accum) {
                    const float4 old = *reinterpret_cast<const float4*>(dst);
                    v = make_float4(old.x + v.x, old.y + v.y, old.z + v.z, old.w + v.w);
                }
                if (P.bias) v = make_float4(v.x + bias4.x, v.y + bias4.y, v.z + bias4.z, v.w + bias4.w);
                if (accum) *reinterpret_cast<float4*>(dst) = v;
                else st_stream(dst, v);
            }
        }
        lgkm_wait0();
        wg_barrier();  // every wave is done with buffer 2
    }
}

// out[c][r] (+)= x[r][c] for x [rows, cols]: 64 x 64 tiles through LDS (65-
// float pitch, so the column reads hit 64 different banks), 256 threads,
// each moving 16 elements; reads and writes run along rows.
constexpr int kTT = 64;

__global__ void __launch_bounds__(256) transpose_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                        float* __restrict__ out, int accumulate, int64_t tiles_c,
                                                        int64_t ntiles) {
    __shared__ float tile[kTT][kTT + 1];
    const int tx = (int)threadIdx.x & 63, ty = (int)threadIdx.x >> 6;
    for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
        const int64_t r0 = (t / tiles_c) * kTT, c0 = (t % tiles_c) * kTT;
#pragma unroll
        for (int i = 0; i < kTT / 4; ++i) {
            const int64_t r = r0 + ty + 4 * i, c = c0 + tx;
            if (r < rows && c < cols) tile[ty + 4 * i][tx] = x[r * cols + c];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kTT / 4; ++i) {
            const int64_t c = c0 + ty + 4 * i, r = r0 + tx;
            if (r < rows && c < cols) {
                float* d = out + c * rows + r;
                const float v = tile[tx][ty + 4 * i];
                *d = accumulate ? *d + v : v;
            }
        }
        __syncthreads();
    }
}

// Split-k second pass: C_p = alpha * sum_s part[p][s] (+ C_p) (+ bias) for
// the kslices partial products of each problem (part: [batch][kslices][m][n],
// contiguous), the slices added in order 0, 1, ... so the result does not
// depend on scheduling.  One thread per 4 consecutive columns of a row.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float* __restrict__ part, int kslices, int64_t m,
                                                            int64_t n, int64_t batch, int64_t batch_inner, float* c,
                                                            int64_t ldc, int64_t sc0, int64_t sc1, float alpha,
                                                            int accumulate, const float* __restrict__ bias,
                                                            int c_vec) {
    const int64_t nq = (n + 3) / 4;
    const int64_t items = batch * m * nq;
    const int64_t mn = m * n;
    const bool part_vec = (n & 3) == 0;
    for (int64_t it = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; it < items;
         it += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = it / nq, j0 = 4 * (it - row * nq);
        const int64_t pb = row / m, i = row - pb * m;
        const float* src = part + pb * kslices * mn + i * n + j0;
        const int cnt = (int)min<int64_t>(4, n - j0);
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < kslices; ++s, src += mn) {
            if (part_vec) {
                const float4 v = *reinterpret_cast<const float4*>(src);
                acc[0] += v.x;
                acc[1] += v.y;
                acc[2] += v.z;
                acc[3] += v.w;
            } else {
                for (int e = 0; e < cnt; ++e) acc[e] += src[e];
            }
        }
        const int64_t po = pb / batch_inner, pi = pb - po * batch_inner;
        float* dst = c + po * sc0 + pi * sc1 + i * ldc + j0;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = alpha * acc[e];
        if (c_vec && cnt == 4) {
            if (accumulate) {
                const float4 old = *reinterpret_cast<const float4*>(dst);
                v[0] = old.x + v[0];
                v[1] = old.y + v[1];
                v[2] = old.z + v[2];
                v[3] = old.w + v[3];
            }
            if (bias) {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = v[e] + bias[j0 + e];
            }
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            for (int e = 0; e < cnt; ++e) {
                float x = v[e];
                if (accumulate) x = dst[e] + x;
                if (bias) x = x + bias[j0 + e];
                dst[e] = x;
            }
        }
    }
}

// Slices per problem for a launch of `work` workgroups (tiles x problems)
// over a k extent of k: a launch that leaves most of the chip idle (fewer
// workgroups than CUs; two fit on each) and has a long k is cut into k
// slices so the workgroups of one pass cover the chip, each slice at least
// kMinSlice long.  1 = no split.
constexpr int64_t kMinSlice = 256;

int64_t choose_kslices(int64_t work, int64_t k) {
    const int64_t cus = num_cus();
    if (work >= cus || k < 4 * kMinSlice) return 1;
    const int64_t s = std::max<int64_t>(2, 2 * cus / work);
    return std::min<int64_t>(s, k / kMinSlice);
}

// ---- rocBLAS for the plain large products ----------------------------------
//
// The vendor library's tuned fp32 kernels beat this file's on large, plain
// products (measured on MI355X, % of the fp32 matrix peak, library /
// gemm_kernel / gemm_dma_kernel: 8192^3 92.9-97.8 / 83-84 / 87-90; the
// [8192, 1024] x [1024, 1024] projections and their weight and input
// gradients 88.9-90.3 / 65-70 / -), lose on bmm's k = 128 forward
// (62.2 / 59.7-63.2 / 72.6 on gemm_dma3_kernel), on its gradients (71 / 74-76 / 80.1) and on
// the attention's per-head products (k = 64 scores 19.7 / 46, n = 64
// contexts 45.7 / 64: two-level batches the library can only take as one
// call per outer batch).  Batched products that gemm_dma_kernel takes run
// there first (launch_gemm).  Unbatched products with m, n >= 128 and
// k >= 256, and the other one-level batches of untransposed products with
// m, n >= 128, k <= 256, no bias and disjoint outputs, go to rocBLAS
// (atomics off: the same bits on every run); the rest to gemm_kernel, and
// while the library route is switched off (wm_gemm_library) every product
// to this file's kernels.  A bias is written into C first and the library adds the
// product to it.  The switch is read once per product; a product racing a
// switch takes one route or the other, whole.
std::atomic<int> g_library{1};  // wm_gemm_library

struct Blas {
    std::mutex mu;
    rocblas_handle h = nullptr;
    bool failed = false;
};

Blas& blas() {
    static Blas* b = new Blas;  // never destroyed: no teardown ordering with the runtime
    return *b;
}

// C rows = bias (one float4 per thread when n, ldc and the stride are
// multiples of 4 and C is aligned; one float otherwise), on a grid covering
// C: the library then adds the product to it (beta = 1).
template <bool VEC>
__global__ void __launch_bounds__(256) bias_rows_kernel(float* __restrict__ c, int64_t m, int64_t n, int64_t ldc,
                                                        int64_t batch, int64_t sc, const float* __restrict__ bias) {
    constexpr int W = VEC ? 4 : 1;
    const int64_t nw = n / W, rows = batch * m;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nw) return;
    const int64_t row = i / nw, j = (i - row * nw) * W;
    const int64_t p = row / m, r = row - p * m;
    float* dst = c + p * sc + r * ldc + j;
    if constexpr (VEC) *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(bias + j);
    else *dst = bias[j];
}

bool fits_int(int64_t v) { return v >= 0 && v <= INT_MAX; }

// The library route for P, or 1 when it does not take P (the caller then
// launches gemm_kernel); WM_OK or an error status when it ran.
int try_library(bool ta, bool tb, const GemmParams& P) {
    if (!g_library.load(std::memory_order_relaxed) || P.kslices > 1) return 1;
    if (P.m < 128 || P.n < 128) return 1;
    if (P.bias && P.accumulate) return 1;
    if (P.batch != 1) {
        // One-level batches of untransposed small-k products (bmm's forward);
        // their gradients and the attention's two-level per-head products
        // measured slower on the library and stay on gemm_kernel.
        if (P.batch_inner != 1 || ta || tb || P.k > 256 || P.bias) return 1;
        if (P.sc0 < P.m * P.ldc) return 1;  // problems sharing output rows stay on gemm_kernel
    } else if (P.k < 256) {
        return 1;
    }
    if (!fits_int(P.m) || !fits_int(P.n) || !fits_int(P.k) || !fits_int(P.lda) || !fits_int(P.ldb) ||
        !fits_int(P.ldc) || !fits_int(P.batch))
        return 1;
    const int64_t sc = 0;
    Blas& B = blas();
    std::lock_guard<std::mutex> lk(B.mu);
    if (B.failed) return 1;
    if (!B.h) {
        if (rocblas_create_handle(&B.h) != rocblas_status_success ||
            rocblas_set_atomics_mode(B.h, rocblas_atomics_not_allowed) != rocblas_status_success ||
            rocblas_set_pointer_mode(B.h, rocblas_pointer_mode_host) != rocblas_status_success) {
            B.failed = true;  // the product still runs, on gemm_kernel
            return 1;
        }
    }
    if (rocblas_set_stream(B.h, stream()) != rocblas_status_success)
        return set_error(WM_ERR_HIP, "wm_gemm: rocblas_set_stream failed");
    float beta = P.accumulate ? 1.0f : 0.0f;
    if (P.bias) {
        const bool vec = P.n % 4 == 0 && P.ldc % 4 == 0 && (P.batch == 1 || sc % 4 == 0) && aligned16(P.c) &&
                         aligned16(P.bias);
        const int64_t items = P.batch * P.m * (vec ? P.n / 4 : P.n);
        const dim3 grid((unsigned)((items + 255) / 256));
        if (vec) launch_kernel(bias_rows_kernel<true>, grid, dim3(256), 0, stream(), P.c, P.m, P.n, P.ldc, P.batch, sc,
                               P.bias);
        else launch_kernel(bias_rows_kernel<false>, grid, dim3(256), 0, stream(), P.c, P.m, P.n, P.ldc, P.batch, sc,
                           P.bias);
        WM_TRY(check_launch("wm_gemm(bias)"));
        beta = 1.0f;
    }
    // Row-major C = op(A) op(B) is column-major C^T = op(B)^T op(A)^T: the
    // row-major buffers read as their column-major transposes.
    const rocblas_operation oa = ta ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_operation ob = tb ? rocblas_operation_transpose : rocblas_operation_none;
    const float alpha = P.alpha;
    const rocblas_status st =
        P.batch == 1
            ? rocblas_sgemm(B.h, ob, oa, (rocblas_int)P.n, (rocblas_int)P.m, (rocblas_int)P.k, &alpha, P.b,
                            (rocblas_int)P.ldb, P.a, (rocblas_int)P.lda, &beta, P.c, (rocblas_int)P.ldc)
            : rocblas_sgemm_strided_batched(B.h, ob, oa, (rocblas_int)P.n, (rocblas_int)P.m, (rocblas_int)P.k,
                                            &alpha, P.b, (rocblas_int)P.ldb, P.sb0, P.a, (rocblas_int)P.lda, P.sa0,
                                            &beta, P.c, (rocblas_int)P.ldc, P.sc0, (rocblas_int)P.batch);
    if (st != rocblas_status_success)
        return set_error(WM_ERR_HIP, std::string("wm_gemm: rocBLAS: ") + rocblas_status_to_string(st));
    return WM_OK;
}

// Whether gemm_dma_kernel takes P: one batch level, every tile interior (m,
// n multiples of 128, k of 64), 16-byte rows, and no k split (gemm_kernel
// splits k when few tiles meet a long k).
bool dma_fits(bool vec, const GemmParams& P, int64_t tiles) {
    return vec && P.batch_inner == 1 && P.m % kTile == 0 && P.n % kTile == 0 && P.k > 0 &&
           P.k % (4 * kDK) == 0 && P.c_aligned && P.ldc % 4 == 0 && (!P.bias || aligned16(P.bias)) &&
           choose_kslices(tiles * P.batch, P.k) == 1;
}

// gemm_dma_kernel for P, or 1 when the grid would not fit (the caller then
// takes the other routes).
int launch_dma(bool ta, bool tb, GemmParams P, int64_t tiles) {
    // Two problems per workgroup while that still leaves two workgroups per CU.
    P.group = P.batch >= 2 && tiles * (P.batch / 2) >= 2 * num_cus() ? 2 : 1;
    const int64_t gy = (P.batch + P.group - 1) / P.group;
    if (gy > 65535) return 1;
    P.kslices = 1;
    P.ksplit = P.k;
    P.sck = 0;
    const dim3 grid((unsigned)tiles, (unsigned)gy);
#define WM_DMA(TA, TB)                                                                                    \
    do {                                                                                                  \
        if (P.k <= 256) launch_kernel((gemm_dma3_kernel<TA, TB>), grid, dim3(kThreads), 0, stream(), P); \
        else launch_kernel((gemm_dma_kernel<TA, TB>), grid, dim3(kThreads), 0, stream(), P);             \
    } while (0)
    if (!ta && !tb) WM_DMA(false, false);
    else if (!ta && tb) WM_DMA(false, true);
    else if (ta && !tb) WM_DMA(true, false);
    else WM_DMA(true, true);
#undef WM_DMA
    return check_launch("wm_gemm(dma)");
}

// Whether gemm_dma32_kernel takes P: A transposed, B not, n = 64 (one
// 64-wide tile), m a multiple of 128, k of 32, 16-byte rows, no k split;
// two batch levels allowed.
bool dma32_fits(bool ta, bool tb, bool vec, const GemmParams& P, int64_t tiles) {
    return ta && !tb && vec && P.batch <= INT_MAX && P.m % kTile == 0 && P.n == 64 && P.k > 0 && P.k % kNK == 0 &&
           P.c_aligned && P.ldc % 4 == 0 && (!P.bias || aligned16(P.bias)) &&
           choose_kslices(tiles * P.batch, P.k) == 1;
}

int launch_dma32(GemmParams P, int64_t tiles) {
    P.group = P.batch >= 2 && tiles * (P.batch / 2) >= 2 * num_cus() ? 2 : 1;
    const int64_t gy = (P.batch + P.group - 1) / P.group;
    if (gy > 65535) return 1;
    P.kslices = 1;
    P.ksplit = P.k;
    P.sck = 0;
    const dim3 grid((unsigned)tiles, (unsigned)gy);
    launch_kernel((gemm_dma32_kernel<true, false>), grid, dim3(kThreads), 0, stream(), P);
    return check_launch("wm_gemm(dma32)");
}

int launch_gemm(bool ta, bool tb, const GemmParams& P0) {
    GemmParams P = P0;
    // 64-wide column tiles for narrow products (attention's per-head products
    // with hd = 64), 128-wide otherwise.
    const bool narrow = P.n <= 64;
    const int64_t bn = narrow ? 64 : 128;
    const int64_t tm = (P.m + kTile - 1) / kTile, tn = (P.n + bn - 1) / bn;
    if (tm * tn > (int64_t)0x7fffffff) return set_error(WM_ERR_INVALID, "wm_gemm: too many tiles");
    P.tiles_m = (int)tm;
    P.tiles_n = (int)tn;
    // The unchecked float4 loads need 16-byte aligned rows in both operands.
    const bool vec = P.lda % 4 == 0 && P.ldb % 4 == 0 && aligned16(P.a) && aligned16(P.b) &&
                     (P.batch == 1 || (P.sa0 % 4 == 0 && P.sa1 % 4 == 0 && P.sb0 % 4 == 0 && P.sb1 % 4 == 0));
    P.c_aligned = aligned16(P.c) && (P.batch == 1 || (P.sc0 % 4 == 0 && P.sc1 % 4 == 0)) ? 1 : 0;
    hipStream_t s = stream();
    P.kslices = 1;
    P.group = 1;
    // Batched products that fit gemm_dma_kernel run there (faster than the
    // library's strided-batched kernels on them); plain ones keep the library
    // unless its route is switched off.
    if (dma_fits(vec, P, tm * tn) && (P.batch > 1 || !g_library.load(std::memory_order_relaxed))) {
        const int r = launch_dma(ta, tb, P, tm * tn);
        if (r != 1) return r;
    }
    if (narrow && dma32_fits(ta, tb, vec, P, tm * tn) &&
        (P.batch > 1 || !g_library.load(std::memory_order_relaxed))) {
        const int r = launch_dma32(P, tm * tn);
        if (r != 1) return r;
    }
    const int lib = try_library(ta, tb, P);
    if (lib != 1) return lib;

    // Split k: the partial products go to a workspace [batch][kslices][m][n]
    // (unscaled, overwritten), and a second pass adds them into C.
    int64_t kslices = choose_kslices(tm * tn * P.batch, P.k);
    Workspace part(0);
    GemmParams F = P;  // the final C, for the second pass
    if (kslices > 1) {
        const int64_t slice = ((P.k + kslices - 1) / kslices + kBK - 1) / kBK * kBK;
        kslices = (P.k + slice - 1) / slice;
        const int64_t mn = P.m * P.n;
        part.p = ws_alloc((size_t)(P.batch * kslices * mn) * sizeof(float));
        if (!part.p) return set_error(WM_ERR_NOMEM, "wm_gemm: split-k workspace");
        P.ksplit = slice;
        P.kslices = (int)kslices;
        P.c = part.as<float>();
        P.ldc = P.n;
        P.sc0 = P.batch_inner * kslices * mn;
        P.sc1 = kslices * mn;
        P.sck = mn;
        P.alpha = 1.0f;
        P.accumulate = 0;
        P.bias = nullptr;
        P.c_aligned = (P.n & 3) == 0 ? 1 : 0;
    } else {
        P.ksplit = P.k;
        P.kslices = 1;
        P.sck = 0;
    }
    dim3 grid((unsigned)(tm * tn), (unsigned)std::min<int64_t>(P.batch * P.kslices, 65535));
#define WM_GEMM(TA, TB, V)                                                                   \
    do {                                                                                     \
        if (narrow) launch_kernel((gemm_kernel<TA, TB, V, 64>), grid, dim3(kThreads), 0, s, P); \
        else launch_kernel((gemm_kernel<TA, TB, V, 128>), grid, dim3(kThreads), 0, s, P);       \
    } while (0)
    if (vec) {
        if (!ta && !tb) WM_GEMM(false, false, true);
        else if (!ta && tb) WM_GEMM(false, true, true);
        else if (ta && !tb) WM_GEMM(true, false, true);
        else WM_GEMM(true, true, true);
    } else {
        if (!ta && !tb) WM_GEMM(false, false, false);
        else if (!ta && tb) WM_GEMM(false, true, false);
        else if (ta && !tb) WM_GEMM(true, false, false);
        else WM_GEMM(true, true, false);
    }
#undef WM_GEMM
    if (P.kslices > 1) {
        WM_TRY(check_launch("wm_gemm"));
        const bool c_vec = F.c_aligned && (F.ldc & 3) == 0;
        const int64_t items = F.batch * F.m * ((F.n + 3) / 4);
        launch_kernel(splitk_reduce_kernel, dim3(grid_for(items, 256)), dim3(256), 0, s, part.as<float>(),
                           P.kslices, F.m, F.n, F.batch, F.batch_inner, F.c, F.ldc, F.sc0, F.sc1, F.alpha,
                           F.accumulate, F.bias, c_vec ? 1 : 0);
    }
    return check_launch("wm_gemm");
}

}  // namespace
}  // namespace wm

using namespace wm;

int wm_gemm(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha, const float* a, int64_t lda,
            const float* b, int64_t ldb, float* c, int64_t ldc, int accumulate, const float* bias, int64_t batch,
            int64_t batch_inner, const int64_t* strides) {
    if (m < 0 || n < 0 || k < 0 || batch < 0) return set_error(WM_ERR_INVALID, "wm_gemm: negative extent");
    if (batch_inner < 1 || (batch > 0 && batch % batch_inner != 0))
        return set_error(WM_ERR_INVALID, "wm_gemm: batch_inner must divide batch");
    if (m == 0 || n == 0 || batch == 0) return WM_OK;
    if (batch > 1 && !strides) return set_error(WM_ERR_INVALID, "wm_gemm: batch > 1 needs strides");
    if (!c || (k > 0 && (!a || !b))) return set_error(WM_ERR_INVALID, "wm_gemm: null pointer");
    const int64_t a_cols = trans_a ? m : k, b_cols = trans_b ? k : n;
    if (lda < std::max<int64_t>(1, a_cols) || ldb < std::max<int64_t>(1, b_cols) || ldc < n)
        return set_error(WM_ERR_INVALID, "wm_gemm: leading dimension smaller than a row");
    WM_CHECK_INIT();
    GemmParams P{};
    P.a = a;
    P.b = b;
    P.c = c;
    P.bias = bias;
    P.m = m;
    P.n = n;
    P.k = k;
    P.lda = lda;
    P.ldb = ldb;
    P.ldc = ldc;
    P.batch = batch;
    P.batch_inner = batch_inner;
    if (strides) {
        P.sa0 = strides[0];
        P.sa1 = strides[1];
        P.sb0 = strides[2];
        P.sb1 = strides[3];
        P.sc0 = strides[4];
        P.sc1 = strides[5];
    }
    P.alpha = alpha;
    P.accumulate = accumulate ? 1 : 0;
    return launch_gemm(trans_a != 0, trans_b != 0, P);
}

int wm_gemm_library(int mode) {
    if (mode == 0 || mode == 1) g_library.store(mode, std::memory_order_relaxed);
    return g_library.load(std::memory_order_relaxed);
}

int wm_matmul(const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* c) {
    return wm_gemm(0, 0, m, n, k, 1.0f, a, std::max<int64_t>(k, 1), b, std::max<int64_t>(n, 1), c, n, 0, nullptr, 1,
                   1, nullptr);
}

int wm_matmul_bwd(const float* g, const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* ga,
                  int accumulate_a, float* gb, int accumulate_b) {
    if (m < 0 || k < 0 || n < 0) return set_error(WM_ERR_INVALID, "wm_matmul_bwd: negative extent");
    const int64_t k1 = std::max<int64_t>(k, 1), n1 = std::max<int64_t>(n, 1);
    if (ga) WM_TRY(wm_gemm(0, 1, m, k, n, 1.0f, g, n1, b, n1, ga, k, accumulate_a, nullptr, 1, 1, nullptr));
    if (gb) WM_TRY(wm_gemm(1, 0, k, n, m, 1.0f, a, k1, g, n1, gb, n, accumulate_b, nullptr, 1, 1, nullptr));
    return WM_OK;
}

int wm_bmm(const float* a, const float* b, int64_t batch, int64_t m, int64_t k, int64_t n, float* c) {
    if (batch < 0 || m < 0 || k < 0 || n < 0) return set_error(WM_ERR_INVALID, "wm_bmm: negative extent");
    const int64_t st[6] = {m * k, 0, k * n, 0, m * n, 0};
    return wm_gemm(0, 0, m, n, k, 1.0f, a, std::max<int64_t>(k, 1), b, std::max<int64_t>(n, 1), c, n, 0, nullptr,
                   batch, 1, st);
}

int wm_bmm_bwd(const float* g, const float* a, const float* b, int64_t batch, int64_t m, int64_t k, int64_t n,
               float* ga, int accumulate_a, float* gb, int accumulate_b) {
    if (batch < 0 || m < 0 || k < 0 || n < 0) return set_error(WM_ERR_INVALID, "wm_bmm_bwd: negative extent");
    const int64_t k1 = std::max<int64_t>(k, 1), n1 = std::max<int64_t>(n, 1);
    if (ga) {
        const int64_t st[6] = {m * n, 0, k * n, 0, m * k, 0};
        WM_TRY(wm_gemm(0, 1, m, k, n, 1.0f, g, n1, b, n1, ga, k, accumulate_a, nullptr, batch, 1, st));
    }
    if (gb) {
        const int64_t st[6] = {m * k, 0, m * n, 0, k * n, 0};
        WM_TRY(wm_gemm(1, 0, k, n, m, 1.0f, a, k1, g, n1, gb, n, accumulate_b, nullptr, batch, 1, st));
    }
    return WM_OK;
}

int wm_transpose2d(const float* x, int64_t rows, int64_t cols, float* out, int accumulate) {
    if (rows < 0 || cols < 0) return set_error(WM_ERR_INVALID, "wm_transpose2d: negative extent");
    if (rows == 0 || cols == 0) return WM_OK;
    if (!x || !out) return set_error(WM_ERR_INVALID, "wm_transpose2d: null pointer");
    if (x == out) return set_error(WM_ERR_INVALID, "wm_transpose2d: in-place transpose is not supported");
    WM_CHECK_INIT();
    const int64_t tiles_c = (cols + kTT - 1) / kTT;
    const int64_t ntiles = ((rows + kTT - 1) / kTT) * tiles_c;
    const unsigned grid = (unsigned)std::min<int64_t>(ntiles, (int64_t)num_cus() * 16);
    launch_kernel(transpose_kernel, dim3(grid), dim3(256), 0, stream(), x, rows, cols, out, accumulate ? 1 : 0,
                       tiles_c, ntiles);
    return check_launch("wm_transpose2d");
}
