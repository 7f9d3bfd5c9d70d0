// gemm.hip -- the prefill projections' GEMM on fp16 MFMA (gfx950):
//   C[m][n] = f16(sum_k A[m][k] * B[n][k]  (+ C[m][n]))
// A: activation rows [M][K], B: weight rows [N][K] (checkpoint layout), both
// K-contiguous; f32 accumulation, one rounding of the f32 result (with the
// residual added in f32 first when accumulating) -- the rounding points of
// the reference's batched projections (cpu_decoder.rs:45-62 batch_dot_acc,
// 398-449; dispatched on the GPU by decoder.rs:3580-4162).
//
// Block tile BM x BN (256 x 256, 192 x 256 down to 64 x 64, chosen per
// shape by a cost model: launch_gemm_f16), K steps of 64, waves in a 2 x WGN grid (WGN = 2:
// four waves, one per SIMD; WGN = 4: eight, two per SIMD, so one wave's
// MFMAs run while the other waits), each wave (BM/2) x (BN/WGN) as tiles of
// v_mfma_f32_32x32x16_f16.  Eight waves measured faster for 256 x 256
// (16384 x 12288 x 2048: 764-820 against 820-861 us), 192 x 256 and
// 128 x 128, four for the smaller tiles.  The two largest tiles run a
// ping-pong schedule of their two wave groups (below); the others run four
// 16-k slices per K step with the next slice's operand reads issued as one
// group ahead of the current slice's MFMAs, and the next step's first reads
// ahead of the last slice's, so no LDS latency is waited for between MFMAs.
// Both operand tiles go global -> LDS by direct copies (buffer_load ... lds,
// one 1 KB block per wave instruction) into NS buffers: the copies of K
// step t+NS are issued as soon as every wave is done with step t's buffers,
// so NS-1 steps are in flight while another is consumed.  Two stages for
// the larger tiles (their LDS then still fits two workgroups per CU up to
// 128 x 128); four for 64 x 64, whose steps are short and latency-bound
// (420 x 2048 x 6144: 47.8 -> 30 us; three or four stages on the larger
// tiles cost the second workgroup per CU and measured slower).  LDS row
// layout (both operands): row r is 128 bytes (64 k), its 16-byte chunk c at slot
// c ^ ((r >> 1) & 7), so an operand read (16 consecutive rows, one chunk)
// covers 16 distinct 16-byte bank groups.  Rows past M are copied from row
// M - 1 (finite values; their outputs are not stored).
// Workgroups are dealt round-robin to the 8 XCDs: when the column blocks
// divide by 8, XCD x takes a contiguous run of them and walks them in groups
// of a few row blocks, so the tiles an XCD runs at one time share a few A
// and B blocks in its L2.
// Results are rounded and stored in place; with the residual they go
// through LDS first, so C is read and written in 8-byte row pieces, all of
// a row tile's residual reads issued before its first store (one memory
// round trip per row tile; 256 x 256 at 4269 x 2048 x 2048: 72 against
// 83.5 us).

#include <algorithm>
#include <cstdlib>

#include "kernels.hpp"

namespace qasr {

namespace {

constexpr int kBK = 64;          // k per step
constexpr int kRowBytes = kBK * 2;  // 128 bytes of one row per step
constexpr int kGroupRows = 4;  // row blocks per group of an XCD's tile walk

__device__ __forceinline__ float16v mfma32(const half8v& a, const half8v& b, const float16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int slot_of(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// s_waitcnt vmcnt(N) lgkmcnt(0): at most N vector memory operations of this
// wave still in flight, and no LDS operation.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0070 | (N & 15) | ((N >> 4) << 14));
}

template <int BM, int BN, int NS, bool ACC, int WGN, bool PP>
__global__ __launch_bounds__(128 * WGN, 1) void gemm_f16_kernel(const f16* __restrict__ A,
                                                                const f16* __restrict__ B,
                                                                f16* __restrict__ C, int M, int N,
                                                                int K) {
    constexpr int kWaves = 2 * WGN;  // 2 x WGN wave grid
    constexpr int WM = BM / 2, WN = BN / WGN;
    constexpr int MT = WM / 32, NT = WN / 32;
    static_assert(MT >= 1 && NT >= 1, "wave tile of whole 32 x 32 MFMA tiles");
    constexpr int ACOPY = BM * kRowBytes / 1024 / kWaves;  // copy instructions per wave and step
    constexpr int BCOPY = BN * kRowBytes / 1024 / kWaves;
    static_assert(ACOPY * kWaves * 1024 == BM * kRowBytes && BCOPY * kWaves * 1024 == BN * kRowBytes,
                  "whole 1 KB copy blocks per wave");
    // NS stages of both operand buffers in one array: the epilogue reuses all
    // of it.
    static_assert(NS >= 2 && NS <= 4, "copy stages");
    __shared__ __attribute__((aligned(16))) f16 smem[NS * (BM + BN) * kBK];
    f16(*As)[BM * kBK] = reinterpret_cast<f16(*)[BM * kBK]>(smem);
    f16(*Bs)[BN * kBK] = reinterpret_cast<f16(*)[BN * kBK]>(smem + NS * BM * kBK);

    // The wave index in a scalar register: the copies' LDS addresses (M0)
    // are then scalar arithmetic, not a vector add and a readfirstlane each.
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int g = lane >> 5, l32 = lane & 31;

    // Block coordinates (see the XCD note above).
    const int nmt = (M + BM - 1) / BM, nnt = N / BN;
    int mt, nt;
    {
        const int bid = blockIdx.x;
        if (nnt % 8 == 0 && gridDim.x == (unsigned)(nmt * nnt)) {
            // XCD x (workgroups x, x + 8, ..) takes column blocks
            // [x nper, (x+1) nper) and walks them in groups of kGroupRows row
            // blocks: group after group, each column block of the group's
            // rows in turn, so the XCD's concurrent tiles share a few A and
            // B blocks in its L2.
            const int x = bid & 7, j = bid >> 3, nper = nnt >> 3;
            const int grp = j / (kGroupRows * nper);
            const int gr = min(kGroupRows, nmt - grp * kGroupRows);
            const int r = j - grp * kGroupRows * nper;
            mt = grp * kGroupRows + r % gr;
            nt = x * nper + r / gr;
        } else {
            mt = bid % nmt;
            nt = bid / nmt;
        }
    }
    const int m0 = mt * BM, n0 = nt * BN;

    const u32x4v ares = make_rsrc_words(A, M * K * 2);
    const u32x4v bres = make_rsrc_words(B, N * K * 2);
    // This thread's copy sources: instruction j of wave w (of W) fills LDS
    // bytes [(W j + w) KB, +1 KB): 16-byte unit p = 64 (W j + w) + lane,
    // row p / 8, slot p % 8, holding chunk slot ^ ((row >> 1) & 7).
    int aoff[ACOPY], boff[BCOPY];
#pragma unroll
    for (int j = 0; j < ACOPY; ++j) {
        const int p = 64 * (kWaves * j + wave) + lane, row = p >> 3;
        const int src = min(m0 + row, M - 1);
        aoff[j] = src * K * 2 + slot_of(row, p & 7) * 16;
    }
#pragma unroll
    for (int j = 0; j < BCOPY; ++j) {
        const int p = 64 * (kWaves * j + wave) + lane, row = p >> 3;
        boff[j] = (n0 + row) * K * 2 + slot_of(row, p & 7) * 16;
    }
    auto copy_step = [&](int t, int buf) {
        const int kb = t * kRowBytes;
#pragma unroll
        for (int j = 0; j < ACOPY; ++j) dma16(ares, aoff[j] + kb, lds_addr(&As[buf][(kWaves * j + wave) * 512]));
#pragma unroll
        for (int j = 0; j < BCOPY; ++j) dma16(bres, boff[j] + kb, lds_addr(&Bs[buf][(kWaves * j + wave) * 512]));
    };

    // Operand reads: A tile i (rows wm WM + 32 i + l32) and B tile i (rows
    // wn WN + 32 i + l32), k-slice ks: chunk 2 ks + g.
    int arow[MT], brow[NT];
#pragma unroll
    for (int i = 0; i < MT; ++i) arow[i] = wm * WM + 32 * i + l32;
#pragma unroll
    for (int i = 0; i < NT; ++i) brow[i] = wn * WN + 32 * i + l32;

    float16v acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = (float16v){};

    const int nk = K / kBK;
    constexpr int kStepCopies = ACOPY + BCOPY;
    static_assert((NS - 1) * kStepCopies <= 63, "vmcnt range");
    // Wait until at most `pending` steps' copies are in flight (the older
    // ones have landed), and for every LDS read of this wave.
    auto wait_steps = [&](int pending) {
        if (NS > 3 && pending >= 3)
            wait_vm_lgkm0<(NS > 3 ? 3 : 0) * kStepCopies>();
        else if (NS > 2 && pending == 2)
            wait_vm_lgkm0<(NS > 2 ? 2 : 0) * kStepCopies>();
        else if (pending == 1)
            wait_vm_lgkm0<kStepCopies>();
        else
            wait_vm_lgkm0<0>();
    };
    const int npro = nk < NS ? nk : NS;  // steps copied ahead
    for (int t = 0; t < npro; ++t) copy_step(t, t);
    wait_steps(npro - 1);
    __syncthreads();

    // Operand registers of two k-slices: slice ks+1's reads are issued as
    // one group ahead of slice ks's MFMAs, so their LDS latency runs under
    // those MFMAs; sched_barrier keeps the compiler from moving a read next
    // to its first use.
    half8v a[2][MT], b[2][NT];
    auto read_slice = [&](const f16* as, const f16* bs, int ks, int q) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            a[q][i] = *(const half8v*)&as[arow[i] * kBK + slot_of(arow[i], 2 * ks + g) * 8];
#pragma unroll
        for (int i = 0; i < NT; ++i)
            b[q][i] = *(const half8v*)&bs[brow[i] * kBK + slot_of(brow[i], 2 * ks + g) * 8];
    };
    auto mfma_slice = [&](int q) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[i][j] = mfma32(a[q][i], b[q][j], acc[i][j]);
    };
    constexpr int kSlices = kBK / 16;
    static_assert(kSlices == 4, "slices 0..2 then the step boundary under slice 3");
    // K step t from buffer t % NS.  All but the last step end with the step
    // boundary (straight-line code, so the compiler's waits track exactly
    // which reads are outstanding).
    auto k_step = [&](int t, bool last) {
        const int buf = t % NS;
        const f16* as = As[buf];
        const f16* bs = Bs[buf];
        // Slice 0's reads were issued under the previous step's last MFMAs:
        // done by now.  Waiting here explicitly keeps the compiler from
        // waiting for the reads issued next, which it would otherwise
        // assume pending across the loop edge.
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
#pragma unroll
        for (int ks = 0; ks + 1 < kSlices; ++ks) {
            read_slice(as, bs, ks + 1, (ks + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            mfma_slice(ks & 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        // Slice 3's operands are in registers.  Once every wave has them
        // (all of its LDS reads of this buffer returned) and step t+1's
        // copies have landed (those of the steps after it may still fly),
        // refill this buffer with step t+NS and read step t+1's slice 0,
        // both under slice 3's MFMAs.
        if (!last) {
            const int newest = t + NS - 1 < nk - 1 ? t + NS - 1 : nk - 1;  // last step copied
            wait_steps(newest - (t + 1));
            __syncthreads();
            if (t + NS < nk) copy_step(t + NS, buf);
            const int nb = (t + 1) % NS;
            read_slice(As[nb], Bs[nb], 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        mfma_slice(1);
        __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (PP) {
        // Ping-pong (the 256 x 256 and 192 x 256 tiles): waves 0-3 (group 0)
        // and 4-7 (group 1), one of each per SIMD, alternate strictly between
        // a read phase (a K step's operands, LDS -> registers, and the copies
        // of the next step) and an MFMA phase (the step's 32 or 24 MFMAs),
        // group 1 one phase behind, every phase ending at a workgroup
        // barrier: while one wave of a SIMD reads, the other feeds the matrix
        // core.  16384 x 12288 x 2048, same box: 256 x 256 714-722 us
        // against 787-795 with group 1's copies moved as described below,
        // and ~800 with the pipelined loop; 192 x 256 801-805 against
        // 827-831.  Half-step phases (twice the barriers) measured in
        // between; 128 x 128 with them (four MFMAs a phase) was slower than
        // its pipelined loop.  Step t is read in global phase 2t by group 0
        // and 2t + 1 by group 1 and multiplied one phase later.  At its read
        // of step t (t >= 1) a wave copies its share of step t + 1 into
        // buffer (t + 1) % 2, which both groups finished reading (step t - 1)
        // in phases 2t - 2 and 2t - 1; step t + 1 is read from phase 2t + 2
        // on, and every wave waits for its own copies (vmcnt) before the
        // barrier that ends phase 2t + 1.  Group 1 thus waits in the phase it
        // copies in; moving its copies into its MFMA phase one step earlier,
        // so that they have two phases, measured 11% slower (the copy
        // instructions then hold up the MFMA issue).  The K order of every
        // output is that of the other tiles, so the bits are too.
        static_assert(NS == 2 && kWaves == 8, "ping-pong: two stages, two waves per SIMD");
        const int grp = __builtin_amdgcn_readfirstlane(wave >> 2);
        half8v pa[kSlices][MT], pb[kSlices][NT];
        // The one-phase offset is a barrier that only group 1 executes at the
        // start and only group 0 at the end.  The condition is uniform per
        // wave (readfirstlane), and every wave executes 2 nk + 1 barriers in
        // all, so each hardware barrier still gathers all eight waves: the
        // k-th barrier of a group-0 wave meets the k-th of a group-1 wave.
        if (grp == 1) __syncthreads();
        for (int t = 0; t < nk; ++t) {
            if (t >= 1 && t + 1 < nk) copy_step(t + 1, (t + 1) & 1);
            const f16* as = As[t & 1];
            const f16* bs = Bs[t & 1];
#pragma unroll
            for (int ks = 0; ks < kSlices; ++ks) {
#pragma unroll
                for (int i = 0; i < MT; ++i)
                    pa[ks][i] = *(const half8v*)&as[arow[i] * kBK + slot_of(arow[i], 2 * ks + g) * 8];
#pragma unroll
                for (int i = 0; i < NT; ++i)
                    pb[ks][i] = *(const half8v*)&bs[brow[i] * kBK + slot_of(brow[i], 2 * ks + g) * 8];
            }
            if (grp == 1) wait_vm_lgkm0<0>();
            __syncthreads();  // (lgkmcnt(0): this phase's reads are in registers)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < kSlices; ++ks)
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int j = 0; j < NT; ++j) acc[i][j] = mfma32(pa[ks][i], pb[ks][j], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
            if (grp == 0) wait_vm_lgkm0<0>();
            __syncthreads();
        }
        if (grp == 0) __syncthreads();
    } else {
        read_slice(As[0], Bs[0], 0, 0);
        for (int t = 0; t + 1 < nk; ++t) k_step(t, false);
        k_step(nk - 1, true);
    }

    // acc[i][j][e]: row wm WM + 32 i + 8 (e / 4) + 4 g + e % 4, column
    // wn WN + 32 j + l32 of the block.
    if constexpr (!ACC) {
        // Plain result: each value rounded and stored where it sits (the
        // stores need no wait, and measured faster than staging them).
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * WM + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
                if (m >= M) continue;
                f16* crow = C + (int64_t)m * N + n0 + wn * WN + l32;
#pragma unroll
                for (int j = 0; j < NT; ++j) crow[32 * j] = (f16)acc[i][j][e];
            }
        return;
    }
    // With the residual: row tile i of the wave (32 rows x WN columns) goes
    // through this wave's LDS region as f32 (rows padded so the two lane
    // halves' writes fall on different banks), then out as row-contiguous
    // 4-column pieces: one 8-byte load of C and one 8-byte store per piece,
    // instead of a dependent 2-byte load per value.
    __syncthreads();  // every wave is past its last operand reads
    constexpr int EP = WN + 8;      // padded row, floats
    constexpr int CPR = WN / 4;     // 4-column pieces per row
    constexpr int RPP = 64 / CPR;   // rows per pass of the wave
    static_assert(kWaves * 32 * EP * 4 <= NS * (BM + BN) * kBK * 2, "epilogue staging fits the operand buffers");
    float* ep = reinterpret_cast<float*>(smem) + wave * (32 * EP);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) ep[(8 * (e >> 2) + 4 * g + (e & 3)) * EP + 32 * j + l32] = acc[i][j][e];
        // Every residual piece of the row tile is requested before the first
        // store (rows past M read row M - 1 and are not stored), so the
        // tile waits for one memory round trip, not one per piece.
        constexpr int kIt = 32 / RPP;
        half4v old[kIt];
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int rr = it * RPP + lane / CPR, cc = (lane % CPR) * 4;
            const int m = min(m0 + wm * WM + 32 * i + rr, M - 1);
            old[it] = *reinterpret_cast<const half4v*>(C + (int64_t)m * N + n0 + wn * WN + cc);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int rr = it * RPP + lane / CPR, cc = (lane % CPR) * 4;
            const float4 v = *(const float4*)&ep[rr * EP + cc];
            const int m = m0 + wm * WM + 32 * i + rr;
            if (m >= M) continue;
            half4v o;
            o[0] = (f16)((float)old[it][0] + v.x);
            o[1] = (f16)((float)old[it][1] + v.y);
            o[2] = (f16)((float)old[it][2] + v.z);
            o[3] = (f16)((float)old[it][3] + v.w);
            *reinterpret_cast<half4v*>(C + (int64_t)m * N + n0 + wn * WN + cc) = o;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): reads done before the next tile's writes
        __builtin_amdgcn_wave_barrier();
    }
}

template <int BM, int BN, int NS = 2, int WGN = 2, bool PP = false>
hipError_t launch_shape(const f16* A, const f16* B, f16* C, int M, int N, int K, bool accumulate,
                        hipStream_t stream) {
    const dim3 grid((unsigned)(((M + BM - 1) / BM) * (N / BN)));
    if (accumulate)
        hipLaunchKernelGGL((gemm_f16_kernel<BM, BN, NS, true, WGN, PP>), grid, dim3(128 * WGN), 0, stream, A, B, C, M, N, K);
    else
        hipLaunchKernelGGL((gemm_f16_kernel<BM, BN, NS, false, WGN, PP>), grid, dim3(128 * WGN), 0, stream, A, B, C, M, N, K);
    return hipGetLastError();
}

}  // namespace

bool gemm_f16_fits(int M, int N, int K) {
    return M > 0 && N > 0 && K > 0 && K % kBK == 0 && N % 256 == 0 &&
           (int64_t)M * K * 2 < (int64_t(1) << 31) && (int64_t)N * K * 2 < (int64_t(1) << 31);
}

hipError_t launch_gemm_f16(const f16* A, const f16* B, f16* C, int M, int N, int K, bool accumulate,
                           int cus, hipStream_t stream) {
    if (!gemm_f16_fits(M, N, K)) return hipErrorInvalidValue;
    // Block tile: the one with the least predicted time.  A candidate fits
    // `occ` workgroups per CU (LDS); its tiles run in rounds of occ x cus,
    // with c = min(occ, ceil(tiles / cus)) of them sharing a CU, and a round
    // takes c x tile area x cost[c - 1], the measured time per unit area of
    // one of c workgroups sharing a CU (small tiles alone on a CU wait on
    // their latencies; a second or third one on the CU hides them).  The
    // costs (256 x 256 = 52) come from sweeps of every candidate over the
    // 1.7B projections at 420 and 4,269 rows and a 16384 x 12288 x 2048
    // product; at each the model picks the fastest tile or one within about
    // 12% of it.  (192 x 256 is for N = 2048 at a few thousand rows: 4,269
    // rows make 184 such tiles, one round, against 136 of 256 x 256.)
    // Every tile accumulates each output over K in the same order, so the
    // choice never changes a result's bits.
    // QASR_GEMM_TILE = 1..6 forces candidate 1..6 (the tests compare them).
    struct Cand { int bm, bn, occ; float cost[3]; };
    constexpr Cand cands[] = {{256, 256, 1, {52.0f, 0.0f, 0.0f}},      // 8 waves, ping-pong
                              {192, 256, 1, {57.0f, 0.0f, 0.0f}},      // 8 waves, ping-pong
                              {128, 128, 2, {72.0f, 60.0f, 0.0f}},     // 8 waves
                              {64, 128, 3, {125.0f, 105.0f, 85.0f}},   // 4 waves
                              {128, 64, 3, {125.0f, 105.0f, 85.0f}},   // 4 waves
                              {64, 64, 2, {170.0f, 112.0f, 0.0f}}};    // 4 waves, 4 stages
    constexpr int kCands = (int)(sizeof cands / sizeof cands[0]);
    const int64_t ncu = std::max(1, cus);
    int best = 0;
    double best_t = 0.0;
    for (int i = 0; i < kCands; ++i) {
        const Cand& c = cands[i];
        const int64_t tiles = (int64_t)((M + c.bm - 1) / c.bm) * (N / c.bn);
        const int64_t rounds = (tiles + c.occ * ncu - 1) / (c.occ * ncu);
        const int conc = (int)std::min<int64_t>(c.occ, (tiles + ncu - 1) / ncu);
        const double t = (double)rounds * conc * c.bm * c.bn * c.cost[conc - 1];
        if (i == 0 || t < best_t) {
            best = i;
            best_t = t;
        }
    }
    const char* forced = std::getenv("QASR_GEMM_TILE");
    const int f = forced ? std::atoi(forced) : 0;
    if (f >= 1 && f <= kCands) best = f - 1;
    switch (best) {
        case 0: return launch_shape<256, 256, 2, 4, true>(A, B, C, M, N, K, accumulate, stream);
        case 1: return launch_shape<192, 256, 2, 4, true>(A, B, C, M, N, K, accumulate, stream);
        case 2: return launch_shape<128, 128, 2, 4>(A, B, C, M, N, K, accumulate, stream);
        case 3: return launch_shape<64, 128, 2, 2>(A, B, C, M, N, K, accumulate, stream);
        case 4: return launch_shape<128, 64, 2, 2>(A, B, C, M, N, K, accumulate, stream);
        default: return launch_shape<64, 64, 4, 2>(A, B, C, M, N, K, accumulate, stream);
    }
}

}  // namespace qasr
