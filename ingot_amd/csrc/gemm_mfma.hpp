// Internal header of the MFMA GEMM: the kernel template and its launcher.
// Each kind's tile configurations are instantiated in their own translation
// unit (gemm_bf16.hip, gemm_bf16x2.hip, gemm_f32.hip, gemm_i8.hip) so the
// library builds them in parallel; gemm_mfma.hip holds the configuration
// tables and the dispatch.
//
// MFMA GEMM for gfx950: Y[M,N] = epilogue(A[M,K] · B[N,K]ᵀ).
//
// One template serves the three math types of the hot path. In every case a
// lane feeds 16 bytes of K into each MFMA step:
//   bf16: v_mfma_f32_16x16x32_bf16 (8 bf16 per lane)
//   f32 : 4 × v_mfma_f32_16x16x4_f32 (one float per lane each)
//   int8: v_mfma_i32_16x16x64_i8 (16 int8 per lane)
// so one LDS layout and one k-slot mapping serve all three. LDS rows are the
// 128-byte k-tiles of A and B rows, unpadded, with 16-byte chunk c of row r
// stored at position c ^ swz(r), which spreads the 16 rows a ds_read_b128
// phase reads over distinct banks. Within an MFMA, lane group g = lane/16 supplies chunk g of
// the current 64-byte half of the k-tile for both operands, so the reduction
// pairs the same k on both sides.
//
// The weight is the first MFMA operand (rows n) and A the second (rows m):
// D[n][m] lands in lane (m%16, n/4) as 4 consecutive n.
//
// Workgroup: WGM×WGN waves (4 or 8), each a (BM/WGM)×(BN/WGN) sub-tile of
// 16×16 MFMA blocks. A and B k-tiles move global → LDS by DMA
// (buffer_load_dwordx4 ... lds): no staging registers, 32-bit range-checked
// buffer offsets, hardware zero-fill past the operand end. An NS-stage LDS
// ring keeps NS-1 k-tiles of DMA in flight while one is multiplied; one
// barrier per k-tile. Tile order is XCD-aware (consecutive tiles of the
// grouped order run on one XCD's L2) and grouped by GROUP_M tile rows. The
// epilogue (bias/C, activation, post scale/shift, or the int8 column-sum
// correction + dequant) runs on the accumulators in registers; its
// per-column and per-row terms are staged in LDS during the prologue.
//
// Reference counterparts: the packed-B sweep + micro-kernel of
// kernels/gemm/gemm.go:280-334,431-490 (f32), PackBBF16/widenPanel
// kernels/gemm/gemm.go:920-962 (bf16 weights), QgemmPackedS8 + VNNI kernel
// kernels/gemm/qgemm.go:246-320 (int8), and the bias/act store epilogue of
// SgemmPackedBEpi kernels/gemm/gemm.go:521-597.

#pragma once

#include <type_traits>

#include "kernels.hpp"

namespace ingot {

namespace {

constexpr int GROUP_M = 4;

template <int KD> struct AccOf { typedef f32x4_t type; };
template <> struct AccOf<KIND_I8> { typedef i32x4_t type; };

template <int KD>
__device__ __forceinline__ void mma16(typename AccOf<KD>::type& acc, const i32x4_t& x, const i32x4_t& y);

template <>
__device__ __forceinline__ void mma16<KIND_BF16>(f32x4_t& acc, const i32x4_t& x, const i32x4_t& y) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, x), __builtin_bit_cast(bf16x8_t, y),
                                                   acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void mma16<KIND_BF16X2>(f32x4_t& acc, const i32x4_t& x, const i32x4_t& y) {
    mma16<KIND_BF16>(acc, x, y);
}

template <>
__device__ __forceinline__ void mma16<KIND_F32>(f32x4_t& acc, const i32x4_t& x, const i32x4_t& y) {
    const f32x4_t xf = __builtin_bit_cast(f32x4_t, x);
    const f32x4_t yf = __builtin_bit_cast(f32x4_t, y);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[0], yf[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[1], yf[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[2], yf[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[3], yf[3], acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void mma16<KIND_I8>(i32x4_t& acc, const i32x4_t& x, const i32x4_t& y) {
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x, y, acc, 0, 0, 0);
}

// The workgroup barrier does not wait for LDS-DMA loads (they count as
// vector-memory loads, not LDS stores), so before it every wave waits until at
// most `groups` of its k-tile DMA groups (G instructions each) are in flight,
// and for all its LDS reads: s_waitcnt vmcnt(groups·G) expcnt(7) lgkmcnt(0).
// DMA groups complete in issue order, so the oldest ones are the ones done.
template <int V>
__device__ __forceinline__ void waitcnt_vm() {
    static_assert(V >= 0 && V < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | 0x70);
}

template <int G, int NS>
__device__ __forceinline__ void wait_dma_groups(int groups) {
    static_assert((NS - 1) * G < 64, "outstanding DMA must fit the 6-bit vmcnt");
    switch (groups) {
        case 0: waitcnt_vm<0>(); break;
        case 1: waitcnt_vm<(NS > 1 ? 1 : 0) * G>(); break;
        case 2: waitcnt_vm<(NS > 2 ? 2 : 0) * G>(); break;
        case 3: waitcnt_vm<(NS > 3 ? 3 : 0) * G>(); break;
        case 4: waitcnt_vm<(NS > 4 ? 4 : 0) * G>(); break;
        case 5: waitcnt_vm<(NS > 5 ? 5 : 0) * G>(); break;
        case 6: waitcnt_vm<(NS > 6 ? 6 : 0) * G>(); break;
        case 7: waitcnt_vm<(NS > 7 ? 7 : 0) * G>(); break;
        default: waitcnt_vm<0>(); break;
    }
}

// Workgroup barrier of the k-loop. The waits it relies on (this wave's DMA
// groups up to the needed k-tile, and its LDS reads) are issued explicitly
// right before it, so it carries no memory fence: a workgroup release fence
// would also wait for every LDS-DMA still in flight and drain the ring. The
// empty asm statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void kloop_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Scheduling template for one half k-step of NM MFMAs, NV DMA loads and ND
// LDS fragment reads: after MFMA i come the next ceil((NV+ND)/NM) memory
// instructions (DMA first), so every load is issued early in the half and the
// remaining MFMAs cover its latency. Instruction classes of
// sched_group_barrier: 0x008 MFMA, 0x020 VMEM read, 0x100 DS read.
template <int NM, int NV, int ND, int I = 0>
__device__ __forceinline__ void interleave() {
    if constexpr (I < NM) {
        constexpr int NMEM = NV + ND;
        constexpr int R = (NMEM + NM - 1) / NM;
        constexpr int lo = I * R < NMEM ? I * R : NMEM;
        constexpr int hi = (I + 1) * R < NMEM ? (I + 1) * R : NMEM;
        constexpr int v = (hi < NV ? hi : NV) - (lo < NV ? lo : NV);
        constexpr int d = (hi - lo) - v;
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x020, v, 0);
        if constexpr (d > 0) __builtin_amdgcn_sched_group_barrier(0x100, d, 0);
        interleave<NM, NV, ND, I + 1>();
    }
}

// The same for three classes of memory instructions issued in order (N1 of
// class C1, then N2 of C2, then N3 of C3) between NM MFMAs. Classes: 0x020
// VMEM read, 0x100 DS read, 0x200 DS write.
template <int NM, int N1, int C1, int N2, int C2, int N3, int C3, int I = 0>
__device__ __forceinline__ void interleave3() {
    if constexpr (I < NM) {
        constexpr int NMEM = N1 + N2 + N3;
        constexpr int R = (NMEM + NM - 1) / NM;
        constexpr int lo = I * R < NMEM ? I * R : NMEM;
        constexpr int hi = (I + 1) * R < NMEM ? (I + 1) * R : NMEM;
        auto cut = [](int x, int a, int b) { return x < a ? 0 : (x > b ? b - a : x - a); };
        constexpr int c1 = cut(hi, 0, N1) - cut(lo, 0, N1);
        constexpr int c2 = cut(hi, N1, N1 + N2) - cut(lo, N1, N1 + N2);
        constexpr int c3 = cut(hi, N1 + N2, NMEM) - cut(lo, N1 + N2, NMEM);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if constexpr (c1 > 0) __builtin_amdgcn_sched_group_barrier(C1, c1, 0);
        if constexpr (c2 > 0) __builtin_amdgcn_sched_group_barrier(C2, c2, 0);
        if constexpr (c3 > 0) __builtin_amdgcn_sched_group_barrier(C3, c3, 0);
        interleave3<NM, N1, C1, N2, C2, N3, C3, I + 1>();
    }
}

// Waits for this wave's LDS accesses only (vmcnt and expcnt left open).
__device__ __forceinline__ void waitcnt_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// LDS chunk swizzle: 16-byte chunk c of tile row r is stored at position
// c ^ swz(r). (r >> 1) & 7 makes the 16 rows a ds_read_b128 phase touches
// land on 16 distinct 16-byte bank groups of a 256-byte bank line.
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

template <int KD> struct KernelArgs { typedef GemmArgsF type; };
template <> struct KernelArgs<KIND_I8> { typedef GemmArgsQ type; };

// RS = 0: k-tiles move global → LDS by DMA into the NS-stage ring (with two
// stages each load is issued one k-tile ahead of its use). RS = 2 (two-stage
// tiles too large for a third LDS stage): the activation k-tiles go by DMA
// into a ring of three slots, and the weight k-tiles through two register
// stages (global → VGPRs → ds_write into two slots), so every load is issued
// two k-tiles ahead. That doubles the time a load has to land, which operands
// coming from HBM need, e.g. behind a cache full of another kernel's output
// (on MI355X a three-stage ring took the DiT MLP-down tile shape from +32%
// to +12% over its warm-cache time).
template <int KD, int BM, int BN, int WGM, int WGN, int NS, int RS = 0>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_kernel(typename KernelArgs<KD>::type p) {
    // The hi/lo kind (A = hi + lo, two bf16 planes) sums each k-tile in one
    // order on every tile: hi first half, hi second half, lo first half, lo
    // second half. Tiles over 128 rows run it as a bf16 GEMM over twice the
    // k-tiles (SPLITK: virtual k-tile 2j is k-tile j of the hi plane, 2j + 1 the
    // same k-tile of the lo plane, both against weight k-tile j), so one
    // activation plane per LDS stage and the bf16 kind's ring; smaller tiles
    // hold both planes in a stage (AP = 2) and multiply in the same order, so a
    // k-tile's weight bytes are loaded once. Every tile of the kind gives the
    // same sums.
    constexpr bool SPLIT = KD == KIND_BF16X2;
    constexpr bool SPLITK = SPLIT && BM > 128;
    constexpr int AP = SPLIT && !SPLITK ? 2 : 1;  // activation planes per LDS stage
    constexpr int NW = WGM * WGN;      // waves per workgroup
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int IA = BM / (8 * NW), IB = BN / (8 * NW);  // 8-row DMA loads per wave per k-tile (A plane, B)
    static_assert(IA * 8 * NW == BM && IB * 8 * NW == BN, "DMA rows must split evenly over the waves");
    constexpr int STAGE = (AP * BM + BN) * KTILE_BYTES;
    static_assert(BM % 32 == 0 && BN % 32 == 0, "tile must be a multiple of 32");
    typedef typename AccOf<KD>::type Acc;

    // NS LDS stages (a ring of k-tiles). Rows are 128 bytes, unpadded; the
    // 16-byte chunk c of row r sits at position c ^ swz(r).
    // Per-column (and, for float outputs, per-row) epilogue terms, staged in
    // LDS at the start so that their loads overlap the first k-tiles' DMA
    // instead of following the k-loop. int8: [0] correction −za′·colsum(+bias),
    // [1] dequant scale, [2] requant multiplier; float: [0] β·C per column
    // (C_ROW, C_SCALAR) and ep_row β·C per row (C_COL); absent terms are −0.0.
    // Columns past N repeat column N−1 (their outputs are not stored).
    constexpr int ECOLS = KD == KIND_I8 ? 3 : 1;
    constexpr int EROWS = KD == KIND_I8 ? 1 : BM;
    static_assert(64 * WGM * WGN >= BN && 64 * WGM * WGN >= EROWS, "one thread per staged column and row");
    constexpr int EXTRA = (ECOLS * BN + EROWS) * 4;
    // Stages larger than 32 KiB start on 64 KiB boundaries when the ring still
    // fits (a stage straddling a 64 KiB boundary slowed the k-loop on MI355X).
    constexpr int SSTRIDE = STAGE > 32768 && NS * 65536 + EXTRA <= 160 * 1024 ? 65536 : STAGE;
    static_assert(NS >= 2 && NS * SSTRIDE + EXTRA <= 160 * 1024, "LDS must fit in 160 KiB");
    // RS: three activation slots of SA bytes at offset 0, two weight slots of
    // SB bytes after them.
    static_assert(RS == 0 || (RS == 2 && NS == 2 && AP == 1), "register staging: two-stage tiles, one activation plane");
    constexpr int SA = AP * BM * KTILE_BYTES, SB = BN * KTILE_BYTES;
    constexpr int RING = RS ? 3 * SA + 2 * SB : NS * SSTRIDE;
    static_assert(RING + EXTRA <= 160 * 1024, "LDS must fit in 160 KiB");
    // One LDS allocation: the ring at offset 0, the staged terms after it.
    __shared__ __attribute__((aligned(1024))) char lds[RING + EXTRA];
    uint32_t(*ep_col)[BN] = (uint32_t(*)[BN])(lds + RING);
    float* ep_row = (float*)(lds + RING + ECOLS * BN * 4);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int wm = wave / WGN, wn = wave % WGN;

    // ---- tile coordinates: XCD-contiguous, then grouped along M ----
    const int nt = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((nt & 7) == 0) bid = (bid & 7) * (nt >> 3) + (bid >> 3);
    const int per_group = GROUP_M * p.tiles_n;
    const int grp = bid / per_group;
    const int first_m = grp * GROUP_M;
    const int gsz = min(p.tiles_m - first_m, GROUP_M);
    const int in_grp = bid - grp * per_group;
    const int m0 = (first_m + in_grp % gsz) * BM;
    const int n0 = (in_grp / gsz) * BN;

    // ---- global → LDS DMA (buffer_load_dwordx4 ... lds) ----
    // One instruction moves 8 rows × 128 bytes: lane l fetches row l/8, global
    // chunk (l%8) ^ (l/8), landing at LDS position l%8 of that row. Loads past
    // a buffer's end return zero (rows >= M; the weight is padded anyway).
    const __amdgpu_buffer_rsrc_t rsa = make_rsrc(p.a + (int64_t)blockIdx.y * p.stride_a_bytes, p.a_bytes);
    const __amdgpu_buffer_rsrc_t rsb = make_rsrc(p.b + (int64_t)blockIdx.y * p.stride_b_bytes, p.b_bytes);
    // Lane l of a DMA covering rows R..R+7 (R a multiple of 8) writes position
    // l%8 of row R + l/8, so it fetches chunk (l%8) ^ swz(R + l/8); swz depends
    // on R only through bit 3 of R, giving two offsets per lane.
    const int lr = lane >> 3, lp = lane & 7;
    uint32_t voff_a[2], voff_b[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = lp ^ swz(h * 8 + lr);
        voff_a[h] = (uint32_t)(lr * p.lda_bytes) + (uint32_t)(c << 4);
        voff_b[h] = (uint32_t)(lr * p.ldb_bytes) + (uint32_t)(c << 4);
    }

    // The whole byte offset (row, plane, k-tile, lane chunk) goes in the
    // range-checked VGPR offset; the SGPR offset stays 0. A k-tile index past
    // the end gets offset 2^31 + row offset (< 2^32, above every extent: the
    // host keeps row offsets below 2^31), so its load fetches nothing and
    // writes zeros: the pipeline below issues one DMA group per k-tile
    // unconditionally.
    const int KT = SPLITK ? 2 * p.kt : p.kt;
    auto dma = [&](char* st, int kt) {
        // plane offsets stay below 2^31 with the rest of the row offset (the host bounds the extent
        // of both planes), so a past-the-end k-tile still lands out of range
        const int kr = SPLITK ? kt >> 1 : kt;
        const uint32_t aofs = SPLITK ? (uint32_t)(kt & 1) * (uint32_t)p.a_plane_bytes : 0u;
        const uint32_t kofs = kt < KT ? (uint32_t)kr * KTILE_BYTES : 0x80000000u;
#pragma unroll
        for (int pl = 0; pl < AP; ++pl)
#pragma unroll
            for (int j = 0; j < IA; ++j) {
                const int r = (j * NW + wave) * 8;
                const uint32_t row = (uint32_t)((m0 + r) * p.lda_bytes) + aofs + (uint32_t)pl * (uint32_t)p.a_plane_bytes + kofs;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, LDS_AS(st + (pl * BM + r) * KTILE_BYTES), 16,
                                                         voff_a[(r >> 3) & 1] + row, 0, 0, 0);
            }
#pragma unroll
        for (int j = 0; j < IB; ++j) {
            const int r = (j * NW + wave) * 8;
            const uint32_t row = (uint32_t)((n0 + r) * p.ldb_bytes) + kofs;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, LDS_AS(st + (AP * BM + r) * KTILE_BYTES), 16,
                                                     voff_b[(r >> 3) & 1] + row, 0, 0, 0);
        }
    };

    // RS: the activation rows by DMA alone, and the weight rows through
    // registers: the same rows, chunks and out-of-range rule as dma(); lwrite_b
    // stores each lane's 16 bytes where its DMA would have landed them.
    auto dma_a = [&](char* st, int kt) {
        const int kr = SPLITK ? kt >> 1 : kt;
        const uint32_t aofs = SPLITK ? (uint32_t)(kt & 1) * (uint32_t)p.a_plane_bytes : 0u;
        const uint32_t kofs = kt < KT ? (uint32_t)kr * KTILE_BYTES : 0x80000000u;
#pragma unroll
        for (int j = 0; j < IA; ++j) {
            const int r = (j * NW + wave) * 8;
            const uint32_t row = (uint32_t)((m0 + r) * p.lda_bytes) + aofs + kofs;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, LDS_AS(st + r * KTILE_BYTES), 16, voff_a[(r >> 3) & 1] + row, 0,
                                                     0, 0);
        }
    };
    auto gload_b = [&](i32x4_t (&dst)[IB], int kt) {
        const int kr = SPLITK ? kt >> 1 : kt;
        const uint32_t kofs = kt < KT ? (uint32_t)kr * KTILE_BYTES : 0x80000000u;
#pragma unroll
        for (int j = 0; j < IB; ++j) {
            const int r = (j * NW + wave) * 8;
            const uint32_t row = (uint32_t)((n0 + r) * p.ldb_bytes) + kofs;
            dst[j] = __builtin_amdgcn_raw_buffer_load_b128(rsb, voff_b[(r >> 3) & 1] + row, 0, 0);
        }
    };
    auto lwrite_b = [&](char* st, const i32x4_t (&src)[IB]) {
#pragma unroll
        for (int j = 0; j < IB; ++j) *(i32x4_t*)(st + ((j * NW + wave) * 8) * KTILE_BYTES + lane * 16) = src[j];
    };

    Acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Acc{0, 0, 0, 0};

    // fragment offsets: lane row fr = lane % 16, chunk (s·4 + lane/16) of the k-tile
    const int fr = lane & 15, fg = lane >> 4;
    int a_off[2], b_off[2];  // within the activation and the weight part of a stage
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int pos = ((s * 4 + fg) ^ swz(fr)) << 4;
        a_off[s] = (wm * WM + fr) * KTILE_BYTES + pos;
        b_off[s] = (wn * WN + fr) * KTILE_BYTES + pos;
    }
    const int axor = p.a_xor ? (int)0x80808080u : 0;

    typedef i32x4_t FragA[AP][TM];
    typedef i32x4_t FragB[TN];
    auto read_frags2 = [&](const char* sa_, const char* sb_, int s, FragA& fa, FragB& fb) {
#pragma unroll
        for (int pl = 0; pl < AP; ++pl)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                fa[pl][i] = *(const i32x4_t*)(sa_ + a_off[s] + (pl * BM + i * 16) * KTILE_BYTES);
                if (KD == KIND_I8) fa[pl][i] ^= axor;
            }
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j] = *(const i32x4_t*)(sb_ + b_off[s] + j * 16 * KTILE_BYTES);
    };
    // a stage of the DMA ring: the activation rows, then the weight rows
    auto read_frags = [&](const char* st, int s, FragA& fa, FragB& fb) {
        read_frags2(st, st + AP * BM * KTILE_BYTES, s, fa, fb);
    };
    // the products of one activation plane and one half k-tile
    auto mma_plane = [&](const i32x4_t (&fa)[TM], const FragB& fb) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) mma16<KD>(acc[i][j], fb[j], fa[i]);
    };

    // Software pipeline over k-tiles: an NS-stage LDS ring filled by DMA NS
    // k-tiles ahead, and two fragment register sets. A k-tile's second-half
    // fragments are read while its first half is multiplied; the barrier sits
    // between the halves (every wave has read the stage; k-tile kt+1 has
    // landed); right after it the consumed stage is refilled with k-tile
    // kt+NS and the next k-tile's first-half fragments are read while the
    // second half is multiplied. Exactly one DMA group is issued per k-tile
    // (past the end: out of range, see dma), so before the barrier each wave
    // waits until at most the NS-2 groups issued after k-tile kt+1's are in
    // flight. The loop body has no branches, so each half is one scheduling
    // region: its memory instructions are spread between its MFMAs
    // (interleave) and sched_barriers keep the wait and the barrier after
    // the half's last MFMA.
    constexpr int G = AP * IA + IB;                               // DMA instructions per wave per k-tile
    constexpr int NFR = AP * TM + TN;                             // LDS fragment reads per half
    // MFMAs per half of the loop body: with both planes in a stage the first
    // half multiplies the hi plane's two half k-tiles, the second the lo plane's
    constexpr int NMF0 = (KD == KIND_F32 ? 4 : 1) * AP * TM * TN;
    constexpr int NMF1 = NMF0;
    FragA fa0, fa1;
    FragB fb0, fb1;
    // The epilogue terms: raw loads issued right after k-tile 0's DMA, the
    // arithmetic and the LDS writes after the rest of the prologue DMA, so the
    // loads' latency overlaps the DMA (a load's value used in the branch that
    // loads it would make the compiler wait for it there, before any DMA).
    uint32_t r0 = 0, r1 = 0, r2 = 0, r3 = 0;
    // RS: the weight's k-tile j lives in rb[j % 2] between its load and its ds_write
    i32x4_t rb0[RS ? IB : 1], rb1[RS ? IB : 1];
    if constexpr (RS) {
        gload_b(rb0, 0);
        dma_a(lds, 0);
    } else {
        dma(lds, 0);
    }
    if (tid < BN) {
        const int nn = min(n0 + tid, p.N - 1);
        if constexpr (KD == KIND_I8) {
            const QEpi& q = p.qepi;
            const int cb = (int)blockIdx.y * q.col_batch;
            r0 = (uint32_t)q.colsum[cb + nn];
            if (q.bias) r1 = (uint32_t)q.bias[cb + nn];
            if (q.yf) r2 = __float_as_uint(q.scale[q.n_scale == 1 ? 0 : nn]);
            r3 = q.rq_mults ? __float_as_uint(q.rq_mults[cb + nn]) : __float_as_uint(q.rq_mult);
        } else {
            const Epi& e = p.epi;
            if (e.c_mode == INGOT_C_ROW || e.c_mode == INGOT_C_SCALAR)
                r0 = __float_as_uint(e.c[e.c_mode == INGOT_C_ROW ? nn : 0]);
        }
    }
    if constexpr (KD != KIND_I8) {
        if (tid < EROWS && p.epi.c_mode == INGOT_C_COL) r1 = __float_as_uint(p.epi.c[min(m0 + tid, p.M - 1)]);
    }
    if constexpr (RS) {
        gload_b(rb1, 1);
        dma_a(lds + SA, 1);
    } else {
#pragma unroll
        for (int s = 1; s < NS; ++s) dma(lds + s * SSTRIDE, s);
    }
    if (tid < BN) {
        if constexpr (KD == KIND_I8) {
            ep_col[0][tid] = (uint32_t)wrap_add(wrap_mul((int32_t)r0, p.qepi.neg_za), (int32_t)r1);
            ep_col[1][tid] = r2;
            ep_col[2][tid] = r3;
        } else {
            const int cm = p.epi.c_mode;
            ep_col[0][tid] = __float_as_uint(cm == INGOT_C_ROW || cm == INGOT_C_SCALAR ? p.epi.beta * __uint_as_float(r0)
                                                                                      : -0.0f);
        }
    }
    if constexpr (KD != KIND_I8) {
        if (tid < EROWS) ep_row[tid] = p.epi.c_mode == INGOT_C_COL ? p.epi.beta * __uint_as_float(r1) : -0.0f;
    } else {
        if (tid < EROWS) ep_row[tid] = -0.0f;
    }
    if constexpr (RS) {
        waitcnt_vm<IB + IA>();  // k-tile 0 of both operands and the epilogue terms landed
        lwrite_b(lds + 3 * SA, rb0);
        gload_b(rb0, 2);
        dma_a(lds + 2 * SA, 2);
        waitcnt_lgkm0();
        kloop_barrier();  // k-tile 0 in LDS; epilogue terms staged
        read_frags2(lds, lds + 3 * SA, 0, fa0, fb0);
    } else {
        wait_dma_groups<G, NS>(NS - 1);
        kloop_barrier();  // k-tile 0 in LDS; epilogue terms staged
        read_frags(lds, 0, fa0, fb0);
    }
    // Register-staged k-loop. At the start of k-tile kt, its activation rows
    // are in slot kt % 3 (kt+1 landed or landing in the next slot, kt+2 in
    // flight into the one after), its weight rows in weight slot kt % 2, and
    // the weight's kt+1 and kt+2 are in flight into rb[(kt+1) % 2] and
    // rb[kt % 2]; kt's first-half fragments are in fa0/fb0. During kt's first
    // half the weight's kt+1 is written to the other weight slot (free since
    // the barrier of kt−1; the compiler waits for those loads only) and that
    // register stage is reloaded with kt+3. Before the barrier each wave waits
    // for its DMA of activation k-tile kt+1: the in-order vector-memory queue
    // then holds only the weight loads of kt+2 and kt+3 and the DMA of kt+2
    // (IB + IA + IB instructions). After it, kt's activation slot is refilled
    // with kt+3. Each load thus has two k-tiles to land. Past the last k-tile
    // the loads are out of range (zeros, never read).
    int sa = 0;  // activation slot of k-tile kt
    auto rs_step = [&](int kt, auto par, i32x4_t (&R)[IB]) {
        constexpr int P = decltype(par)::value;  // kt % 2
        char* acur = lds + sa * SA;
        const int sa1 = sa == 2 ? 0 : sa + 1;
        char* bcur = lds + 3 * SA + P * SB;
        char* bnxt = lds + 3 * SA + (1 - P) * SB;
        read_frags2(acur, bcur, 1, fa1, fb1);
        mma_plane(fa0[0], fb0);
        lwrite_b(bnxt, R);
        gload_b(R, kt + 3);
        interleave3<NMF0, NFR, 0x100, IB, 0x200, IB, 0x020>();
        __builtin_amdgcn_sched_barrier(0);
        waitcnt_vm<IB + IA + IB>();
        kloop_barrier();  // kt read by every wave; kt+1 of both operands in LDS
        __builtin_amdgcn_sched_barrier(0);
        dma_a(acur, kt + 3);
        read_frags2(lds + sa1 * SA, bnxt, 0, fa0, fb0);  // after the last k-tile: unused
        mma_plane(fa1[0], fb1);
        interleave<NMF1, IA, NFR>();
        __builtin_amdgcn_sched_barrier(0);
        sa = sa1;
    };
    if constexpr (RS) {
        int kt = 0;
        for (; kt + 1 < KT; kt += 2) {
            rs_step(kt, std::integral_constant<int, 0>(), rb1);
            rs_step(kt + 1, std::integral_constant<int, 1>(), rb0);
        }
        if (kt < KT) rs_step(kt, std::integral_constant<int, 0>(), rb1);
    }
    int st = 0;  // ring slot of k-tile kt
    for (int kt = 0; kt < (RS ? 0 : KT); ++kt) {
        char* cur = lds + st * SSTRIDE;
        const int st1 = st + 1 == NS ? 0 : st + 1;
        read_frags(cur, 1, fa1, fb1);
        mma_plane(fa0[0], fb0);
        if constexpr (AP == 2) mma_plane(fa1[0], fb1);
        interleave<NMF0, 0, NFR>();
        __builtin_amdgcn_sched_barrier(0);
        wait_dma_groups<G, NS>(NS - 2);
        kloop_barrier();  // cur fully read by every wave; k-tile kt+1 landed
        __builtin_amdgcn_sched_barrier(0);
        dma(cur, kt + NS);
        if constexpr (AP == 2) {
            // lo first half (kept from before the refill), then lo second half
            i32x4_t lo0[TM];
            FragB b0;
#pragma unroll
            for (int i = 0; i < TM; ++i) lo0[i] = fa0[1][i];
#pragma unroll
            for (int j = 0; j < TN; ++j) b0[j] = fb0[j];
            read_frags(lds + st1 * SSTRIDE, 0, fa0, fb0);  // after the last k-tile: unused
            mma_plane(lo0, b0);
            mma_plane(fa1[1], fb1);
        } else {
            read_frags(lds + st1 * SSTRIDE, 0, fa0, fb0);  // after the last k-tile: unused
            mma_plane(fa1[0], fb1);
        }
        interleave<NMF1, G, NFR>();
        __builtin_amdgcn_sched_barrier(0);
        st = st1;
    }
    // The tail's out-of-range DMA groups land before the workgroup ends (its
    // LDS may be handed to the next workgroup).
    waitcnt_vm<0>();

    // ---- epilogue: straight from the accumulators ----
    // Lane (r, g) holds Y[m][n..n+3] of each 16×16 block (m = block row + r,
    // n = block column + 4g): one 16-byte store per block, 16 rows × 64 bytes
    // per store instruction. Each epilogue step is a wave-uniform branch
    // around an unrolled pass over all accumulators, so accumulators are only
    // indexed statically and the per-element code is branch-free.
    const int r = lane & 15;
    const int g4 = (lane >> 4) * 4;
    const int row0 = m0 + wm * WM + r;
    const int col0 = n0 + wn * WN + g4;
    const int64_t ybatch = (int64_t)blockIdx.y * p.stride_y;
    // 16-byte stores need an aligned row start (n is always a multiple of 4 here)
    uintptr_t ybase;
    bool y16;  // bf16 output: 8-byte stores (else 16-byte)
    if constexpr (KD == KIND_I8) {
        ybase = (uintptr_t)(p.qepi.yi ? p.qepi.yi + ybatch : nullptr) | (uintptr_t)(p.qepi.yf ? p.qepi.yf + ybatch : nullptr) |
                (uintptr_t)(p.qepi.yq ? (uint8_t*)p.qepi.yq + ybatch : nullptr);
        y16 = false;
    } else {
        ybase = (uintptr_t)p.y + ybatch * (p.epi.y_bf16 ? 2 : 4);
        y16 = p.epi.y_bf16;
    }
    const bool vec_ok = (ybase & (y16 ? 7 : 15)) == 0 && (p.ldy & 3) == 0;

    if constexpr (KD == KIND_I8) {
        const QEpi& q = p.qepi;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = col0 + j * 16;
            if (n >= p.N) continue;
            const int lc = n - n0;  // column within the tile (a multiple of 4)
            const i32x4_t corr = *(const i32x4_t*)&ep_col[0][lc];
            const f32x4_t sc = *(const f32x4_t*)&ep_col[1][lc];
            const f32x4_t mu = *(const f32x4_t*)&ep_col[2][lc];
            const bool full = n + 3 < p.N;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int m = row0 + i * 16;
                if (m >= p.M) continue;
                const int64_t o = ybatch + (int64_t)m * p.ldy + n;
                int32_t v[4];
                float f[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = wrap_add(acc[i][j][e], corr[e]);
                    f[e] = (float)wrap_add(v[e], -q.dq_zp) * sc[e];
                }
                if (full && vec_ok) {
                    // non-temporal: the int32 / f32 outputs are 4× the operand
                    // bytes, and leaving them dirty in L2 makes the end of the
                    // kernel wait for their write-back (on MI355X the 1024 × 768
                    // → 3072 MatMulInteger + dequant took 9.0 µs per call with
                    // plain stores, 7.2–7.5 with these)
                    if (q.yi) __builtin_nontemporal_store(i32x4_t{v[0], v[1], v[2], v[3]}, (i32x4_t*)(q.yi + o));
                    if (q.yf) __builtin_nontemporal_store(f32x4_t{f[0], f[1], f[2], f[3]}, (f32x4_t*)(q.yf + o));
                } else {
                    for (int e = 0; e < 4 && n + e < p.N; ++e) {
                        if (q.yi) q.yi[o + e] = v[e];
                        if (q.yf) q.yf[o + e] = f[e];
                    }
                }
                if (q.yq) {
                    // the product and the sum rounded separately (no contraction into
                    // an FMA), then half-to-even and saturation
#pragma clang fp contract(off)
                    uint32_t packed = 0;
                    uint8_t qb[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float t = (float)v[e] * mu[e];
                        const float r = rintf(t + q.rq_zy);
                        const int iv = q.yq_u8 ? (r <= 0.f ? 0 : (r >= 255.f ? 255 : (int)r))
                                               : (r <= -128.f ? -128 : (r >= 127.f ? 127 : (int)r));
                        qb[e] = (uint8_t)iv;
                        packed |= (uint32_t)qb[e] << (8 * e);
                    }
                    uint8_t* yq = (uint8_t*)q.yq;
                    if (q.conv_p > 0) {
                        // one byte per channel plane; lanes r = 0..15 fill 16 consecutive pixels
                        const int img = m / q.conv_p;
                        const int64_t ob = ybatch + (int64_t)img * q.conv_img + (m - img * q.conv_p);
                        for (int e = 0; e < 4 && n + e < p.N; ++e) yq[ob + (int64_t)(n + e) * q.conv_p] = qb[e];
                    } else if (full && vec_ok) {
                        *(uint32_t*)(yq + o) = packed;
                    } else {
                        for (int e = 0; e < 4 && n + e < p.N; ++e) yq[o + e] = qb[e];
                    }
                }
            }
        }
    } else {
        // v = post(act(alpha·acc + beta·C)): the C term is split into a
        // per-column part (C_ROW, C_SCALAR), a per-row part (C_COL) and a
        // per-element load (C_FULL); absent terms are −0.0, the exact
        // additive identity (x + −0 = x, signed zeros included), and an
        // absent post step is ·1 + −0. One activation switch around
        // straight-line code keeps accumulators out of branch joins.
        const Epi& e = p.epi;
        const float nz = -0.0f;
        f32x4_t cn[TN];
        float cm[TM];
#pragma unroll
        for (int j = 0; j < TN; ++j) cn[j] = *(const f32x4_t*)&ep_col[0][col0 - n0 + j * 16];
#pragma unroll
        for (int i = 0; i < TM; ++i) cm[i] = ep_row[row0 - m0 + i * 16];
        const bool cfull = e.c_mode == INGOT_C_FULL;
        const float ps = e.post ? e.post_scale : 1.f, pt = e.post ? e.post_shift : nz;
        void* y = p.y;
        auto store_all = [&](auto act) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int m = row0 + i * 16;
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int n = col0 + j * 16;
                    f32x4_t c4 = cn[j];
                    if (cfull) {
                        const int64_t mc = min(m, p.M - 1);
#pragma unroll
                        for (int q = 0; q < 4; ++q) c4[q] = e.beta * e.c[mc * e.ldc + min(n + q, p.N - 1)];
                    }
                    f32x4_t v;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float x = e.alpha * acc[i][j][q] + c4[q] + cm[i];
                        v[q] = apply_act(x, decltype(act)::value, e.act_alpha, e.act_beta) * ps + pt;
                    }
                    if (m < p.M && n < p.N) {
                        const int64_t o = ybatch + (int64_t)m * p.ldy + n;
                        if (n + 3 < p.N && vec_ok) {
                            if (e.y_bf16) {
                                const uint32_t lo = f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
                                const uint32_t hi = f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
                                *(uint2*)((uint16_t*)y + o) = make_uint2(lo, hi);
                            } else {
                                *(f32x4_t*)((float*)y + o) = v;
                            }
                        } else {
                            for (int q = 0; q < 4 && n + q < p.N; ++q) store_y(y, o + q, v[q], e);
                        }
                    }
                }
            }
        };
        switch (e.act) {
#define INGOT_ACT_CASE(A) \
    case A: store_all(std::integral_constant<int, A>()); break;
            INGOT_ACT_CASE(INGOT_ACT_RELU)
            INGOT_ACT_CASE(INGOT_ACT_GELU_ERF)
            INGOT_ACT_CASE(INGOT_ACT_GELU_TANH)
            INGOT_ACT_CASE(INGOT_ACT_SIGMOID)
            INGOT_ACT_CASE(INGOT_ACT_SILU)
            INGOT_ACT_CASE(INGOT_ACT_HARDSWISH)
            INGOT_ACT_CASE(INGOT_ACT_HARDSIGMOID)
            INGOT_ACT_CASE(INGOT_ACT_CLIP)
            INGOT_ACT_CASE(INGOT_ACT_LEAKYRELU)
#undef INGOT_ACT_CASE
            default: store_all(std::integral_constant<int, INGOT_ACT_NONE>()); break;
        }
    }
}

template <int KD, int BM, int BN, int WGM, int WGN, int NS, int RS = 0>
hipError_t launch_one(const GemmArgs& a, int batch, hipStream_t st) {
    // the grid was sized from the configuration table: it must be exactly this tile's
    if ((int64_t)a.tiles_m * BM < a.M || (int64_t)(a.tiles_m - 1) * BM >= a.M || (int64_t)a.tiles_n * BN < a.N ||
        (int64_t)(a.tiles_n - 1) * BN >= a.N)
        return hipErrorInvalidValue;
    dim3 grid(a.tiles_m * a.tiles_n, batch);
    typename KernelArgs<KD>::type k;
    static_cast<GemmCore&>(k) = a;
    if constexpr (KD == KIND_I8)
        k.qepi = a.qepi;
    else
        k.epi = a.epi;
    hipLaunchKernelGGL((gemm_kernel<KD, BM, BN, WGM, WGN, NS, RS>), grid, dim3(64 * WGM * WGN), 0, st, k);
    return hipGetLastError();
}

}  // namespace

// One launcher per kind (the tile configurations of gemm_configs, by index).
hipError_t launch_gemm_bf16(int cfg, const GemmArgs& a, int batch, hipStream_t st);
hipError_t launch_gemm_bf16x2(int cfg, const GemmArgs& a, int batch, hipStream_t st);
hipError_t launch_gemm_f32(int cfg, const GemmArgs& a, int batch, hipStream_t st);
hipError_t launch_gemm_i8(int cfg, const GemmArgs& a, int batch, hipStream_t st);

}  // namespace ingot
