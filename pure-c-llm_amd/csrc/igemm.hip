// igemm.hip -- u8 x s8 -> int32 GEMM on the CDNA4 int8 matrix cores
// (v_mfma_i32_32x32x32_i8), with the dequantising epilogue.
//
// Reference semantics (gemm_bench.c:212-285): activations are u8 with a +128
// offset, weights s8; vpdpbusd forms acc = sum Au*Bq and the kernel subtracts
// corr = 128*colsum, i.e. v = sum (Au-128)*Bq (gemm_bench.c:216-217, 274).
// The i8 MFMA is signed x signed, so A is re-centred with Au ^ 0x80, which is
// exactly Au-128 as an s8 byte: the MFMA then produces v directly, bit-exact,
// with no column-sum pass. An optional per-column int32 offset reproduces a
// caller-supplied `corr` (off = 128*colsum - corr). Dequant
// (gemm_bench.c:272-275, dq precomputed at :378) is fp32 RNE in the same
// order: C = float(v) * dq with dq = sb[n] or sa[m]*sb[n].
//
// Layouts: A is M x K u8 row-major (K-contiguous). B is pre-packed N x Kp s8
// (K-contiguous per output column, zero from K to Kp = roundup(K, 256); the
// reference packs its weights offline too, gemm_bench.c:218-220).
//
// Data movement. Tiles of BM (BN) rows x 128 bytes of K go from HBM straight
// into LDS with global_load_lds_dwordx4: each wave instruction moves 64 x 16
// bytes into 1 KB of consecutive LDS, no VGPRs involved, so STAGES tiles can
// be in flight at once. Per-lane source offsets are computed once; per tile
// only a scalar base moves. A K tile is consumed from LDS by 16-byte fragment
// reads (ds_read_b128) feeding the MFMA; A fragments are re-centred by XOR in
// registers one step ahead of their use.
//
// LDS layout: row r of a tile is 128 bytes = 8 chunks of 16 bytes; logical
// chunk c lives at physical chunk c ^ ((r >> 1) & 7). The LDS serves a
// ds_read_b128 16 lanes at a time out of 64 four-byte banks (16 chunk slots
// per 256 bytes), and 16 consecutive lanes read 16 consecutive rows at the
// same logical chunk: rows 2q and 2q+1 differ in the 256-byte half, pairs
// differ in the swizzled chunk, so the 16 reads hit 16 distinct slots. A DMA
// instruction fills 8 whole rows, lanes choosing their global chunk so the
// physical layout comes out swizzled.
//
// Schedule. A tile is 4 steps of one 32-byte k-chunk; a step is TM x TN
// MFMAs. The fragments of step s+2 are read while step s multiplies (a ring
// of 4 register slots), and the work of a step -- its LDS reads, the DMA
// issue, the wait and XOR for step s+1 -- is spread over the gaps between its
// MFMAs, so the wave keeps issuing while each MFMA runs (a wave issues in
// order: work bunched between two MFMAs would idle the matrix core).
//
// Synchronisation: one s_barrier per K tile, in step 2. Before it, each wave
// waits (lgkmcnt) for its own fragment reads of the tile, which by then are
// all issued, and (vmcnt) for its own DMA of the next tile, leaving STAGES-2
// younger tiles in flight; after it, the current tile's stage is refilled and
// the next tile's first fragments are read while the current tile's last
// MFMAs run. No fence is used: a release fence would wait for every
// outstanding load and drain the pipeline.
//
// Tails are handled without per-element branches: rows past M (N) are clamped
// to the last row and only feed outputs that are never stored. K is a
// multiple of 256: the launcher pads A (with 0x80, i.e. zero) otherwise, and
// packed weight rows are Kp = roundup(K, 256) >= K bytes, zero past K.
//
// K order: the 32x32x32 MFMA takes 16 bytes per lane; lane group g = lane/32
// supplies logical chunk 2kc+g of the tile for A and for B alike, so the
// integer sum is the same whatever order the hardware reduces it in.
#include "internal.h"

namespace pcl {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) int32_t gint32_t;
typedef __attribute__((address_space(1))) float gfloat_t;
typedef __attribute__((address_space(1))) unsigned gu32_t;

constexpr int IG_BK = 128;  // bytes of K per tile
constexpr int IG_KC = 4;    // 32-byte MFMA k-chunks (steps) per tile

// s_waitcnt immediate for "vmcnt <= n", leaving expcnt and lgkmcnt unchecked.
constexpr int waitcnt_vm(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (15 << 8); }

// Fragment reads from LDS are issued by inline assembly and waited for
// explicitly. The compiler's own wait insertion turns every LDS wait into
// lgkmcnt(0) once LDS DMA instructions are in flight, which would serialise
// each read with the MFMAs it is meant to overlap. Contract: a register
// written by lds_read16 is not touched until lds_wait<n>() has retired the
// read and reg_fence() has been applied to it (the fence orders every later
// use after the wait).
template <int OFF>
__device__ __forceinline__ void lds_read16(v4i &r, unsigned addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds_read offset field");
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
}
template <int OFF>
__device__ __forceinline__ void lds_write16(unsigned addr, const v4i &v) {
    static_assert(OFF >= 0 && OFF < 65536, "ds_write offset field");
    asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(addr), "v"(v), "i"(OFF));
}
template <int N>
__device__ __forceinline__ void lds_wait() {
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N < 15 ? N : 15));
}
__device__ __forceinline__ void reg_fence(v4i &r) { asm volatile("" : "+v"(r)); }

__device__ __forceinline__ unsigned lds_addr(const void *p) {
    return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// Work items of one step, spread over the gaps after its MFMAs (see the
// schedule note above). Step kinds: 0/1 plain, 2 hand-over, 3 after it.
template <int NR, int D1, int D2>
struct StepPlan {
    // items other than the final wait+XOR
    static constexpr int body(int kc) { return kc < 2 ? NR : (kc == 2 ? 1 + D1 + NR : NR + D2); }
    static constexpr bool has_x(int kc) { return kc != 2; }  // step 2 XORs inside its hand-over
};

// BM x BN output tile per workgroup of WM x WN waves; STAGES-deep LDS ring
// of 128-byte K tiles; OCC workgroups are meant to share a CU (the LDS ring
// is sized for it and the register budget is capped accordingly).
// Requires M*lda and N*ldb below 2^32 (32-bit per-lane DMA offsets).
template <int BM, int BN, int WM, int WN, int STAGES, int OCC, int OUT, int NTS>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(
    (OCC * WM * WN + 3) / 4))) void igemm_mfma_kernel(const uint8_t *__restrict__ A, long lda,
                                                     const int8_t *__restrict__ B, long ldb,
                                                     const int32_t *__restrict__ col_off,
                                                     const float *__restrict__ sa,
                                                     const float *__restrict__ sb,
                                                     void *__restrict__ Cv, long ldc, int M, int N,
                                                     int K) {
    constexpr int NW = WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int NM = TM * TN;                       // MFMAs per step
    constexpr int NR = TM + TN;                       // fragment reads per step
    // K tile: 128 bytes; a row of a tile is CH = 8 16-byte chunks
    constexpr int BK = IG_BK;
    constexpr int CH = BK / 16;
    constexpr int RPI = 1024 / BK;  // tile rows per DMA instruction
    constexpr int SIZE_A = BM * BK, SIZE_B = BN * BK;
    constexpr int STAGE = SIZE_A + SIZE_B;
    constexpr int INST_A = BM / (RPI * NW), INST_B = BN / (RPI * NW);  // DMA per wave per tile
    constexpr int LOADS = INST_A + INST_B;
    constexpr int D1 = (LOADS + 1) / 2, D2 = LOADS - D1;
    using Plan = StepPlan<NR, D1, D2>;
    static_assert(TM >= 1 && TN >= 1 && STAGES >= 2, "bad tile configuration");
    static_assert(BM % (RPI * NW) == 0 && BN % (RPI * NW) == 0, "tile rows must split over the waves");
    static_assert((STAGES - 1) * LOADS <= 63, "vmcnt range");
    static_assert(STAGES * STAGE * OCC <= 160 * 1024, "LDS budget of a CU");

    __shared__ __attribute__((aligned(1024))) int8_t lds[STAGES * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int r32 = lane & 31, g = lane >> 5;

    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int bm, bn;
    tile_coords(xcd_remap(blockIdx.x, nbm * nbn), nbm, nbn, 8, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;
    const int wrow0 = m0 + wm * WTM, wcol0 = n0 + wn * WTN;

    // Epilogue operands are loaded before the first K tile (clamped indexes,
    // no branches), so their latency hides behind the main loop. Lane l keeps
    // the values of column wcol0 + 32j + l%32 and of row wrow0 + 32i + l%32.
    float sbv[TN], sav[TM];
    unsigned offv[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int colc = min(wcol0 + j * 32 + r32, N - 1);
        sbv[j] = (OUT != 0) ? sb[colc] : 0.f;
        offv[j] = (OUT != 0 && col_off) ? (unsigned)col_off[colc] : 0u;
    }
#pragma unroll
    for (int i = 0; i < TM; i++) sav[i] = (OUT == 2) ? sa[min(wrow0 + i * 32 + r32, M - 1)] : 0.f;

    // Materialise the epilogue's scalar arguments now: a scalar load still
    // in flight when the K loop starts would make every LDS wait in the loop
    // a full lgkmcnt(0) (scalar loads complete out of order).
    void *C_out = Cv;
    long ld_out = ldc;
    asm volatile("" : "+s"(C_out), "+s"(ld_out));

    // DMA instruction d (A for d < INST_A, else B) of this wave fills the RPI
    // tile rows from rb = RPI*(j*NW + wave); lane l loads row rb + l/CH at the
    // logical chunk whose swizzled slot is l%CH. voff is the lane's byte
    // offset in its operand at k = 0; ldso the instruction's uniform LDS offset.
    const int8_t *A8 = reinterpret_cast<const int8_t *>(A);
    unsigned voff[LOADS];
    int ldso[LOADS];
#pragma unroll
    for (int d = 0; d < LOADS; d++) {
        const bool isA = d < INST_A;
        const int rb = ((isA ? d : d - INST_A) * NW + wave) * RPI;
        const int r = rb + lane / CH;
        const int c = (lane % CH) ^ ((r >> 1) & (CH - 1));
        const int grow = min((isA ? m0 : n0) + r, (isA ? M : N) - 1);
        voff[d] = (unsigned)grow * (unsigned)(isA ? lda : ldb) + (unsigned)(c * 16);
        ldso[d] = (isA ? 0 : SIZE_A) + rb * BK;
    }
    const int nk = K / BK;
    const unsigned lds0 = lds_addr(lds);

    // One DMA instruction of tile t: a scalar base (operand + BK t) plus the
    // lane's fixed offset; no per-tile vector arithmetic. K is a multiple of
    // BK (the launcher pads A otherwise), so every chunk is in its row.
    auto dma = [&](int t, int d) {
        const bool isA = d < INST_A;
        const int8_t *base = (isA ? A8 : B) + (long)t * BK;
        __builtin_amdgcn_global_load_lds((const void *)(base + voff[d]),
                                         (lds_void_t *)(lds + (t % STAGES) * STAGE + ldso[d]), 16, 0,
                                         0);
    };

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0;

    // Fragment ring: slot c holds k-chunk c (32-byte chunk c of the tile) of
    // the current or the next tile. Lane l reads row l%32 of each 32-row
    // block at 16-byte chunk 2c + l/32; the row swizzle depends on l%32 only.
    v4i fa[IG_KC][TM], fb[IG_KC][TN];
    const int swz = (r32 >> 1) & (CH - 1);
    unsigned offa[IG_KC], offb[IG_KC];
#pragma unroll
    for (int c = 0; c < IG_KC; c++) {
        const int chunk = ((2 * c + g) ^ swz) << 4;
        offa[c] = (wm * WTM + r32) * BK + chunk;
        offb[c] = SIZE_A + (wn * WTN + r32) * BK + chunk;
    }
    // read item r (A fragments first) of slot C from the stage at `base`
    auto read_item = [&](unsigned base, auto C, auto R) {
        constexpr int c = decltype(C)::value, r = decltype(R)::value;
        if constexpr (r < TM) lds_read16<r * 32 * BK>(fa[c][r], base + offa[c]);
        else lds_read16<(r - TM) * 32 * BK>(fb[c][r - TM], base + offb[c]);
    };
    // slot C has landed (after the caller's wait): fence it and re-centre A
    auto xor_slot = [&](auto C) {
        constexpr int c = decltype(C)::value;
        static_for<0, TM>([&](auto I) { reg_fence(fa[c][I.value]); });
        static_for<0, TN>([&](auto J) { reg_fence(fb[c][J.value]); });
        static_for<0, TM>([&](auto I) { fa[c][I.value] ^= (int)0x80808080u; });
    };

    // Prologue: every stage is filled; tile 0 is waited for; slots 0 and 1
    // are read and slot 0 is re-centred.
#pragma unroll
    for (int t = 0; t < STAGES; t++)
        if (t < nk) static_for<0, LOADS>([&](auto D) { dma(t, D.value); });
    if (nk >= STAGES) __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 1) * LOADS));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __builtin_amdgcn_s_barrier();
    static_for<0, NR>([&](auto R) { read_item(lds0, IC<0>{}, R); });
    static_for<0, NR>([&](auto R) { read_item(lds0, IC<1>{}, R); });
    lds_wait<NR>();
    xor_slot(IC<0>{});

    for (int kt = 0; kt < nk; kt++) {
        const unsigned cur = lds0 + (kt % STAGES) * STAGE;
        const unsigned nxt = lds0 + ((kt + 1) % STAGES) * STAGE;
        const bool refill = kt + STAGES < nk;
        static_for<0, IG_KC>([&](auto KC) {
            constexpr int kc = KC.value;
            constexpr int pc = (kc + 2) % IG_KC;  // slot being prefetched
            const unsigned pbase = (kc + 2 < IG_KC) ? cur : nxt;
            constexpr int NB = Plan::body(kc);
            constexpr int G = NM > 1 ? NM - 1 : 1;  // gaps that take body items
            // body item b of this step
            auto item = [&](auto Bi) {
                constexpr int b = decltype(Bi)::value;
                if constexpr (kc < 2) {
                    read_item(pbase, IC<pc>{}, IC<b>{});
                } else if constexpr (kc == 2) {
                    if constexpr (b == 0) {
                        // Hand-over to tile kt+1: this wave's reads of tile
                        // kt are complete and its DMA of tile kt+1 has
                        // landed; after the barrier the same holds for every
                        // wave, so tile kt's stage may be refilled.
                        lds_wait<0>();
                        xor_slot(IC<3>{});
                        if (kt + STAGES - 1 < nk)
                            __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 2) * LOADS));
                        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
                        __builtin_amdgcn_s_barrier();
                    } else if constexpr (b <= D1) {
                        if (refill) dma(kt + STAGES, b - 1);
                    } else {
                        read_item(pbase, IC<pc>{}, IC<b - 1 - D1>{});
                    }
                } else {
                    if constexpr (b < NR) read_item(pbase, IC<pc>{}, IC<b>{});
                    else if (refill) dma(kt + STAGES, D1 + b - NR);
                }
            };
            static_for<0, NM>([&](auto Q) {
                constexpr int q = Q.value, i = q % TM, j = q / TM;
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[kc][i], fb[kc][j], acc[i][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (q < G) {
                    static_for<q * NB / G, (q + 1) * NB / G>(item);
                }
                if constexpr (q == G - 1 && Plan::has_x(kc)) {
                    // slot kc+1 is older than this step's NR reads
                    lds_wait<NR>();
                    xor_slot(IC<(kc + 1) % IG_KC>{});
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        });
    }
    lds_wait<0>();  // the last prefetch reads retire before their registers are reused
    // Epilogue: register v of lane l holds row rl = (v/4)*8 + (l/32)*4 + v%4,
    // column l%32 of each 32x32 block. The row scale of rl is fetched from
    // lane rl by a cross-lane permute (no memory access); stores carry no
    // waits, so they stream out back to back.
    // A tile wholly inside C stores without bounds checks; one address per
    // output row serves the TN columns of the row (immediate offsets).
    auto store_tile = [&](auto CHECK) {
        constexpr bool chk = decltype(CHECK)::value != 0;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            float rs[16];
#pragma unroll
            for (int v = 0; v < 16; v++) rs[v] = (OUT == 2) ? __shfl(sav[i], (v >> 2) * 8 + g * 4 + (v & 3)) : 0.f;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = wrow0 + i * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
                if (chk && row >= M) continue;
                const long ro = (long)row * ld_out + wcol0 + r32;
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    if (chk && wcol0 + j * 32 + r32 >= N) continue;
                    const long o = ro + j * 32;
                    // Outputs up to 256 MiB are written with streaming (non-temporal)
                    // stores: write-back through L2 would leave the whole
                    // output dirty in L2 for the end-of-kernel release to
                    // flush. Large outputs stream better through L2.
                    if (OUT == 0) {
                        if constexpr (NTS) __builtin_nontemporal_store(acc[i][j][v], (gint32_t *)C_out + o);
                        else ((gint32_t *)C_out)[o] = acc[i][j][v];
                    } else {
                        const int32_t vv = (int32_t)((unsigned)acc[i][j][v] + offv[j]);
                        const float dq = (OUT == 2) ? rs[v] * sbv[j] : sbv[j];
                        if constexpr (NTS) __builtin_nontemporal_store((float)vv * dq, (gfloat_t *)C_out + o);
                        else ((gfloat_t *)C_out)[o] = (float)vv * dq;
                    }
                }
            }
        }
    };
    if (m0 + BM <= M && n0 + BN <= N)
        store_tile(IC<0>{});
    else
        store_tile(IC<1>{});
}

// ---------------------------------------------------------------------------
// Warp-specialised persistent variant for output-bound shapes (K small next
// to the fp32 output, e.g. K = 1024): WM x WN consumer waves (one K group,
// 128-byte K tiles, the four-step schedule of igemm_mfma_kernel) plus four
// producer waves. The producers issue every LDS DMA and do every vmcnt wait,
// so a consumer never waits on vmcnt: the output stores of one tile drain
// while the consumers multiply the next (on gfx9 one counter tracks loads
// and stores, so a wave that also loaded would wait for its own stores).
// Each workgroup loops over output tiles slot, slot + gridDim, ...; the
// K-tile stream runs across tile boundaries through a STAGES-deep ring. The
// epilogue operands of a tile (sb, col_off, sa) are copied into LDS by the
// producers (4-byte DMA), three tiles deep.
//
// Barrier protocol (all waves run the same number of s_barrier): P0 after
// the prologue, then one barrier B(g) per K tile g in the consumers' step 2.
// Before B(g) the producers have waited for K tile g+1 (leaving g+2 .. in
// flight) and every consumer has issued and retired its reads of K tile g;
// after it the producers refill tile g's stage with tile g + STAGES.
//
// Row classes (P > 1 or col_shift): an output whose rows do not all start on
// a 128-byte line (a pitch like the 50257-float vocabulary head, or a base
// off a line) would have every 32-float store chunk straddle two lines, and
// lines written in two parts by different waves or workgroups halve the HBM
// write rate. Rows r and r + P start at the same offset within a line when
// P * ldc is a multiple of 32 floats, so a tile takes BM rows of one class
// (rows cls, cls + P, cls + 2P, ...) and a column window shifted left by the
// class's offset: its every 32-float chunk is then one whole line. Row
// class cls = bm % P, class-local rows bm / P * BM ...; column tile bn covers
// [bn*BN - csh, bn*BN - csh + BN) with csh = (C's element offset within a
// line + cls * ldc) mod 32. P = 1 without col_shift is the plain tiling.
template <int BM, int BN, int WM, int WN, int STAGES, int NWP, int OUT, int NTS>
__global__ __launch_bounds__(64 * (WM * WN + NWP)) __attribute__((amdgpu_waves_per_eu(
    (WM * WN + NWP + 3) / 4))) void igemm_wp_kernel(const uint8_t *__restrict__ A, long lda,
                                                      const int8_t *__restrict__ B, long ldb,
                                                      const int32_t *__restrict__ col_off,
                                                      const float *__restrict__ sa,
                                                      const float *__restrict__ sb,
                                                      void *__restrict__ Cv, long ldc, int M, int N,
                                                      int K, int P, int col_shift, int gm) {
    constexpr int NWC = WM * WN, BK = IG_BK;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
    constexpr int NM = TM * TN, NR = TM + TN;
    constexpr int CH = BK / 16, RPI = 1024 / BK;  // 8 chunks per row, 8 rows per DMA instruction
    constexpr int SIZE_A = BM * BK, STAGE = (BM + BN) * BK;
    constexpr int PIA = BM / (RPI * NWP), PIB = BN / (RPI * NWP), PL = PIA + PIB;
    constexpr int SCL = 2 * BN + BM + 128;  // floats per tile: sb, col_off, sa, spare
    constexpr int NS = OUT != 0 ? 8 / NWP : 0;  // epilogue-operand DMA instructions per producer
    constexpr int LDS_BYTES = STAGES * STAGE + 3 * SCL * 4;
    static_assert(BM % (RPI * NWP) == 0 && BN % (RPI * NWP) == 0, "rows per producer");
    static_assert(NWP == 2 || NWP == 4 || NWP == 8, "producer waves");
    static_assert(TM >= 1 && TN >= 1 && STAGES >= 2, "tile configuration");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget of a CU");
    static_assert(BN == 128 && BM <= 256, "epilogue operands: two 64-lane DMA per producer wave");
    static_assert((STAGES - 1) * (PL + NS) <= 63, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) int8_t lds[LDS_BYTES];
    float *scl = reinterpret_cast<float *>(lds + STAGES * STAGE);  // [3 tiles][sb | col_off | sa]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int Mc = (M + P - 1) / P;  // rows of the largest class
    const int nbm = P * ((Mc + BM - 1) / BM), nbn = (N + (col_shift ? 31 : 0) + BN - 1) / BN;
    const int ntiles = nbm * nbn;
    const int cb0 = col_shift ? (int)((reinterpret_cast<unsigned long>(Cv) >> 2) & 31) : 0;
    const int nb = gridDim.x;
    const int slot = xcd_remap(blockIdx.x, nb);
    const int my_tiles = slot < ntiles ? (ntiles - 1 - slot) / nb + 1 : 0;
    const int nk = K / BK;
    const int G = my_tiles * nk;  // K tiles this workgroup streams
    if (G == 0) return;           // uniform: no barrier is left unmatched
    // tile i of this workgroup: row class, class-local first row, first column
    // (negative for the window that holds a class's first partial line)
    auto tile_origin = [&](int i, int &cls, int &r0, int &n0) {
        int bm, bn;
        tile_coords(i * nb + slot, nbm, nbn, gm, bm, bn);
        cls = bm % P;
        r0 = bm / P * BM;
        n0 = bn * BN - (col_shift ? (int)((cb0 + (long)cls * ldc) & 31) : 0);
    };

    if (wave >= NWC) {
        // ------------------------------------------------------ producers
        const int pw = wave - NWC;
        const int8_t *A8 = reinterpret_cast<const int8_t *>(A);
        unsigned voff[PL];
        int ldso[PL];
        // Output tile i starts: per-lane source offsets of its A rows and B
        // columns (swizzled chunk order, as in igemm_mfma_kernel), and the
        // 4-byte DMA of its epilogue operands into LDS buffer i % 3: eight
        // 64-lane pieces (sb 0-1, col_off 2-3, sa 4-7), producer pw issuing
        // pieces [pw*NS, pw*NS + NS); an absent piece (no col_off, no sa, sa
        // rows past BM) loads sb again into the spare slot, so every producer
        // issues the same count.
        auto begin_tile = [&](int i) {
            int cls, r0, n0;
            tile_origin(i, cls, r0, n0);
#pragma unroll
            for (int d = 0; d < PL; d++) {
                const bool isA = d < PIA;
                const int rb = ((isA ? d : d - PIA) * NWP + pw) * RPI;
                const int r = rb + lane / CH;
                const int c = (lane % CH) ^ ((r >> 1) & (CH - 1));
                // rows past the output re-read the last row; columns outside
                // [0, N) the nearest one (their results are never stored)
                const int grow = isA ? min(cls + P * (r0 + r), M - 1) : max(min(n0 + r, N - 1), 0);
                voff[d] = (unsigned)grow * (unsigned)(isA ? lda : ldb) + (unsigned)(c * 16);
                ldso[d] = (isA ? 0 : SIZE_A) + rb * BK;
            }
            if (OUT != 0) {
                float *dst = scl + (i % 3) * SCL;
#pragma unroll
                for (int h = 0; h < NS; h++) {
                    const int piece = pw * NS + h;
                    const float *src = sb + max(min(n0 + (piece & 1) * 64 + lane, N - 1), 0);
                    float *to = dst + 2 * BN + BM + (piece & 1) * 64;  // spare slot
                    if (piece < 2) {
                        to = dst + piece * 64;
                    } else if (piece < 4) {
                        if (col_off) {
                            src = reinterpret_cast<const float *>(col_off) +
                                  max(min(n0 + (piece - 2) * 64 + lane, N - 1), 0);
                            to = dst + BN + (piece - 2) * 64;
                        }
                    } else if (OUT == 2 && (piece - 4) * 64 < BM) {
                        src = sa + min(cls + P * (r0 + (piece - 4) * 64 + lane), M - 1);
                        to = dst + 2 * BN + (piece - 4) * 64;
                    }
                    __builtin_amdgcn_global_load_lds((const void *)src, (lds_void_t *)to, 4, 0, 0);
                }
            }
        };
        int di = 0, dk = 0;  // output tile and K tile of the next DMA
        // issue K tile di*nk + dk; returns whether it carried epilogue operands
        auto dma_next = [&]() -> bool {
            const bool first = dk == 0;
            if (first) begin_tile(di);
            const long koff = (long)dk * BK;
            int8_t *stage = lds + ((di * nk + dk) % STAGES) * STAGE;
#pragma unroll
            for (int d = 0; d < PL; d++)
                __builtin_amdgcn_global_load_lds((const void *)((d < PIA ? A8 : B) + koff + voff[d]),
                                                 (lds_void_t *)(stage + ldso[d]), 16, 0, 0);
            if (++dk == nk) {
                dk = 0;
                di++;
            }
            return first && NS > 0;
        };
        // hist bit j: the j-th most recently issued K-tile DMA also carried
        // epilogue operands (NS more vmcnt entries than PL, issued before its
        // PL loads). Waits count them exactly: "the NY youngest K tiles may
        // still fly" is vmcnt <= NY * PL + NS * (those of them that carried
        // operands), so a tile boundary does not drain the DMA queue.
        unsigned hist = 0;
        auto wait_younger = [&](auto NYC) {
            constexpr int ny = decltype(NYC)::value;
            const int c = __builtin_popcount(hist & ((1u << ny) - 1));
            static_for<0, ny + 1>([&](auto Cc) {
                constexpr int cc = decltype(Cc)::value;
                if (c == cc) __builtin_amdgcn_s_waitcnt(waitcnt_vm(ny * PL + cc * NS));
            });
        };
        // prologue: K tiles 0 .. STAGES-1; P0 once K tile 0 has landed
#pragma unroll
        for (int t = 0; t < STAGES; t++)
            if (t < G) hist = (hist << 1) | (dma_next() ? 1u : 0u);
        if (G >= STAGES) wait_younger(IC<STAGES - 1>{});
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __builtin_amdgcn_s_barrier();
        // before B(g) K tiles g+1 .. g+STAGES-1 have been issued, oldest first
        for (int g = 0; g < G; g++) {
            // K tile g+1 has landed; the STAGES-2 younger ones may still fly
            if (g + STAGES - 1 < G) wait_younger(IC<STAGES - 2>{});
            else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            __builtin_amdgcn_s_barrier();  // B(g)
            if (g + STAGES < G) hist = (hist << 1) | (dma_next() ? 1u : 0u);  // into stage g % STAGES
        }
        return;
    }

    // ---------------------------------------------------------- consumers
    const int wm = wave / WN, wn = wave % WN;
    const int r32 = lane & 31, lg = lane >> 5;
    void *C_out = Cv;
    long ld_out = ldc;
    int Mv = M, Nv = N;
    asm volatile("" : "+s"(C_out), "+s"(ld_out), "+s"(Mv), "+s"(Nv));
    const unsigned lds0 = lds_addr(lds);

    v16i acc[TM][TN];
    v4i fa[IG_KC][TM], fb[IG_KC][TN];
    const int swz = (r32 >> 1) & (CH - 1);
    unsigned offa[IG_KC], offb[IG_KC];
#pragma unroll
    for (int c = 0; c < IG_KC; c++) {
        const int chunk = ((2 * c + lg) ^ swz) << 4;
        offa[c] = (wm * WTM + r32) * BK + chunk;
        offb[c] = SIZE_A + (wn * WTN + r32) * BK + chunk;
    }
    auto read_item = [&](unsigned base, auto C, auto R) {
        constexpr int c = decltype(C)::value, r = decltype(R)::value;
        if constexpr (r < TM) lds_read16<r * 32 * BK>(fa[c][r], base + offa[c]);
        else lds_read16<(r - TM) * 32 * BK>(fb[c][r - TM], base + offb[c]);
    };
    auto xor_slot = [&](auto C) {
        constexpr int c = decltype(C)::value;
        static_for<0, TM>([&](auto I) { reg_fence(fa[c][I.value]); });
        static_for<0, TN>([&](auto J) { reg_fence(fb[c][J.value]); });
        static_for<0, TM>([&](auto I) { fa[c][I.value] ^= (int)0x80808080u; });
    };

    __builtin_amdgcn_s_barrier();  // P0
    static_for<0, NR>([&](auto R) { read_item(lds0, IC<0>{}, R); });
    static_for<0, NR>([&](auto R) { read_item(lds0, IC<1>{}, R); });
    lds_wait<NR>();
    xor_slot(IC<0>{});

    int gk = 0;  // K tile index in this workgroup's stream
    for (int i = 0; i < my_tiles; i++) {
#pragma unroll
        for (int a = 0; a < TM; a++)
#pragma unroll
            for (int b = 0; b < TN; b++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[a][b][v] = 0;

        for (int kt = 0; kt < nk; kt++, gk++) {
            const unsigned cur = lds0 + (gk % STAGES) * STAGE;
            const unsigned nxt = lds0 + ((gk + 1) % STAGES) * STAGE;
            static_for<0, IG_KC>([&](auto KC) {
                constexpr int kc = KC.value;
                constexpr int pc = (kc + 2) % IG_KC;
                const unsigned pbase = (kc + 2 < IG_KC) ? cur : nxt;
                constexpr int NB = kc == 2 ? 1 + NR : NR;
                constexpr int GP = NM > 1 ? NM - 1 : 1;
                auto item = [&](auto Bi) {
                    constexpr int b = decltype(Bi)::value;
                    if constexpr (kc == 2) {
                        if constexpr (b == 0) {
                            // B(gk): this wave's reads of K tile gk are retired
                            lds_wait<0>();
                            xor_slot(IC<3>{});
                            __builtin_amdgcn_s_barrier();
                        } else {
                            read_item(pbase, IC<pc>{}, IC<b - 1>{});
                        }
                    } else {
                        read_item(pbase, IC<pc>{}, IC<b>{});
                    }
                };
                static_for<0, NM>([&](auto Q) {
                    constexpr int q = Q.value, a = q % TM, b = q / TM;
                    acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[kc][a], fb[kc][b], acc[a][b], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    if constexpr (q < GP) {
                        static_for<q * NB / GP, (q + 1) * NB / GP>(item);
                    }
                    if constexpr (q == GP - 1 && kc != 2) {
                        lds_wait<NR>();
                        xor_slot(IC<(kc + 1) % IG_KC>{});
                    }
                    __builtin_amdgcn_sched_barrier(0);
                });
            });
        }

        // Epilogue (layout as in igemm_mfma_kernel); operands from LDS. The
        // stores carry no wait: they drain while the next tile is multiplied.
        int cls, r0, n0;
        tile_origin(i, cls, r0, n0);
        const int wrow0 = r0 + wm * WTM, wcol0 = n0 + wn * WTN;  // class-local row
        const float *sc = scl + (i % 3) * SCL;
        float sbv[TN];
        unsigned offv[TN];
#pragma unroll
        for (int b = 0; b < TN; b++) {
            const int cl = wn * WTN + b * 32 + r32;
            sbv[b] = (OUT != 0) ? sc[cl] : 0.f;
            offv[b] = (OUT != 0 && col_off) ? reinterpret_cast<const unsigned *>(sc)[BN + cl] : 0u;
        }
        // a tile wholly inside C stores without bounds checks, one address per
        // output row for its TN columns
        auto store_tile = [&](auto CHECK) {
            constexpr bool chk = decltype(CHECK)::value != 0;
#pragma unroll
            for (int a = 0; a < TM; a++) {
#pragma unroll
                for (int vq = 0; vq < 4; vq++) {
                    typedef float v4f_t __attribute__((ext_vector_type(4)));
                    const v4f_t rs4 = (OUT == 2) ? *reinterpret_cast<const v4f_t *>(
                                                       sc + 2 * BN + wm * WTM + a * 32 + vq * 8 + lg * 4)
                                                 : v4f_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int v = vq * 4 + e;
                        const int row = cls + P * (wrow0 + a * 32 + vq * 8 + lg * 4 + e);
                        if (chk && row >= Mv) continue;
                        const long ro = (long)row * ld_out + wcol0 + r32;
#pragma unroll
                        for (int b = 0; b < TN; b++) {
                            const int col = wcol0 + b * 32 + r32;
                            if (chk && (col < 0 || col >= Nv)) continue;
                            const long o = ro + b * 32;
                            if (OUT == 0) {
                                if constexpr (NTS) __builtin_nontemporal_store(acc[a][b][v], (gint32_t *)C_out + o);
                                else ((gint32_t *)C_out)[o] = acc[a][b][v];
                            } else {
                                const int32_t vv = (int32_t)((unsigned)acc[a][b][v] + offv[b]);
                                const float dq = (OUT == 2) ? rs4[e] * sbv[b] : sbv[b];
                                if constexpr (NTS) __builtin_nontemporal_store((float)vv * dq, (gfloat_t *)C_out + o);
                                else ((gfloat_t *)C_out)[o] = (float)vv * dq;
                            }
                        }
                    }
                }
            }
        };
        if (cls + P * (r0 + BM - 1) < Mv && n0 >= 0 && n0 + BN <= Nv)
            store_tile(IC<0>{});
        else
            store_tile(IC<1>{});
    }
}

// ---------------------------------------------------------------------------
// Producer/consumer kernel for grids of about one 128x128 output tile per CU
// (2048^3, the K = 4096 down projection, the attention output projection):
// one tile per workgroup, eight consumer waves on v_mfma_i32_16x16x64_i8,
// NWP producer waves, a STAGES-deep ring of 128-byte K tiles.
//
// What bounds it. A 128x128 tile consumes 32 KB of operands per 128-byte K
// tile. The L2 -> LDS stream of these grids moves ~22 TB/s into LDS (about
// 88 GB/s per CU; measured with the DMA alone), so the loop is bound by the
// operand feed, and the feed runs at the shader clock, which the matrix cores
// pull down to 1.4-1.8 GHz on random operands. Two choices follow:
//  * every consumer wave reads a whole K tile's fragments into registers one
//    tile ahead, so a stage can be refilled as soon as the MFMAs of its tile
//    begin: with a 3- or 4-deep ring two or three K tiles are in flight;
//  * the 16x16x64 instruction: a loop of it alone holds ~2.05 GHz on random
//    bytes against ~1.7 GHz for the 32x32x32 form at the same work per clock.
// KGR = 1: 4x2 consumer waves of 32x64, each over the whole K tile (12
// fragment reads per K tile). KGR = 2: two K groups of 2x2 waves of 64x64,
// group g multiplies the 64 k-bytes g of every K tile (8 reads: a third fewer
// LDS bytes) and the groups' partial tiles are added once at the end through
// the freed ring. Integer sums are exact in any order: both forms are
// bit-identical to the integer definition.
//
// Barrier protocol (every wave runs the same sequence): P0 once K tile 0 has
// landed; then B(kt) for each K tile, after the first MFMA of tile kt in the
// consumers. Before B(kt) every consumer has retired its reads of K tile kt
// (issued during tile kt-1) and the producers have waited for K tile kt+1;
// after it the producers refill tile kt's stage with tile kt + STAGES and the
// consumers read tile kt+1. With KGR = 2 one more barrier orders the exchange.
template <int STAGES, int NWP, int KGR, int OUT, int NTS>
__global__ __launch_bounds__(64 * (8 + NWP)) __attribute__((amdgpu_waves_per_eu(
    (8 + NWP + 3) / 4))) void igemm_kg_kernel(const uint8_t *__restrict__ A, long lda,
                                             const int8_t *__restrict__ B, long ldb,
                                             const int32_t *__restrict__ col_off,
                                             const float *__restrict__ sa,
                                             const float *__restrict__ sb,
                                             void *__restrict__ Cv, long ldc, int M, int N,
                                             int K) {
    constexpr int BM = 128, BN = 128, BK = IG_BK, CH = BK / 16, RPI = 1024 / BK;
    constexpr int SIZE_A = BM * BK, STAGE = (BM + BN) * BK;
    constexpr int PIA = BM / (RPI * NWP), PIB = BN / (RPI * NWP), PL = PIA + PIB;
    constexpr int LDS_BYTES = STAGES * STAGE;
    constexpr int XW = 8192;  // exchange bytes per consumer wave (half of a 64x64 int32 tile)
    static_assert(NWP == 2 || NWP == 4, "producer waves");
    static_assert(KGR == 1 || KGR == 2, "K groups");
    static_assert(STAGES >= 3 && LDS_BYTES <= 160 * 1024, "ring");
    static_assert(LDS_BYTES >= 8 * XW, "the exchange reuses the ring");
    static_assert((STAGES - 1) * PL <= 63, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) int8_t lds[LDS_BYTES];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int bm, bn;
    tile_coords(xcd_remap(blockIdx.x, nbm * nbn), nbm, nbn, 8, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;
    const int nk = K / BK;

    if (wave >= 8) {
        // ------------------------------------------------------ producers
        const int pw = wave - 8;
        const int8_t *A8 = reinterpret_cast<const int8_t *>(A);
        unsigned voff[PL];
        int ldso[PL];
#pragma unroll
        for (int d = 0; d < PL; d++) {
            const bool isA = d < PIA;
            const int rb = ((isA ? d : d - PIA) * NWP + pw) * RPI;
            const int r = rb + lane / CH;
            const int c = (lane % CH) ^ ((r >> 1) & (CH - 1));
            const int grow = min((isA ? m0 : n0) + r, (isA ? M : N) - 1);
            voff[d] = (unsigned)grow * (unsigned)(isA ? lda : ldb) + (unsigned)(c * 16);
            ldso[d] = (isA ? 0 : SIZE_A) + rb * BK;
        }
        auto dma = [&](int t) {
            int8_t *stage = lds + (t % STAGES) * STAGE;
            const long koff = (long)t * BK;
#pragma unroll
            for (int d = 0; d < PL; d++)
                __builtin_amdgcn_global_load_lds((const void *)((d < PIA ? A8 : B) + koff + voff[d]),
                                                 (lds_void_t *)(stage + ldso[d]), 16, 0, 0);
        };
        // Prologue: tiles 0 and 1, P0 once tile 0 has landed, then the rest of
        // the ring (issued all at once, tile 0 would queue behind the whole ring
        // in L2 and the first MFMA would wait for it).
        dma(0);
        if (nk > 1) {
            dma(1);
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(PL));
        } else {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        }
        __builtin_amdgcn_s_barrier();  // P0
#pragma unroll
        for (int t = 2; t < STAGES; t++)
            if (t < nk) dma(t);
        for (int kt = 0; kt < nk; kt++) {
            // K tile kt+1 has landed; tiles kt+2 .. kt+STAGES-1 may still fly
            if (kt + STAGES - 1 < nk) __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 2) * PL));
            else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            __builtin_amdgcn_s_barrier();  // B(kt)
            if (kt + STAGES < nk) dma(kt + STAGES);
        }
        if constexpr (KGR == 2) __builtin_amdgcn_s_barrier();  // exchange
        return;
    }

    // ---------------------------------------------------------- consumers
    constexpr int WM = KGR == 2 ? 2 : 4;
    constexpr int WTM = BM / WM, WTN = 64;     // wave tile
    constexpr int NBM = WTM / 16, NBN = WTN / 16;  // 16x16 blocks
    constexpr int KS = 2 / KGR;                // 64-byte k-steps per wave per K tile
    constexpr int NFA = KS * NBM, NFB = KS * NBN, NF = NFA + NFB;
    constexpr int NM = KS * NBM * NBN;         // MFMAs per K tile
    const int kg = KGR == 2 ? wave >> 2 : 0;
    const int wm = KGR == 2 ? (wave >> 1) & 1 : wave >> 1, wn = wave & 1;

    // Epilogue operands first (clamped, no branches): their loads complete
    // under the K loop. Lane l holds column l%16 of each 16-wide block and
    // rows 4(l/16) + r of each stored 16-row block (the rows kg*32 .. kg*32+31
    // of the wave tile).
    void *C_out = Cv;
    long ld_out = ldc;
    int Mv = M, Nv = N;
    asm volatile("" : "+s"(C_out), "+s"(ld_out), "+s"(Mv), "+s"(Nv));
    const int wrow0 = m0 + wm * WTM, wcol0 = n0 + wn * WTN;
    const int lcol = lane & 15;
    float sbv[NBN];
    unsigned offv[NBN];
#pragma unroll
    for (int j = 0; j < NBN; j++) {
        const int colc = min(wcol0 + j * 16 + lcol, Nv - 1);
        sbv[j] = (OUT != 0) ? sb[colc] : 0.f;
        offv[j] = (OUT != 0 && col_off) ? (unsigned)col_off[colc] : 0u;
    }
    float sav[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const int r = kg * 32 + (q >> 2) * 16 + 4 * (lane >> 4) + (q & 3);
        sav[q] = (OUT == 2) ? sa[min(wrow0 + r, Mv - 1)] : 0.f;
    }

    const unsigned lds0 = lds_addr(lds);
    // Fragment offsets in a stage: lane (r16, g4) reads row r16 of a 16-row
    // block at 16-byte chunk 4(kg*KS + s) + g4 of the 128-byte K tile. Rows are
    // stored with chunk c at c ^ ((row >> 1) & 7); blocks start at multiples of
    // 16 rows, so the swizzle depends on the lane only.
    const int lrow = lane & 15, lgrp = lane >> 4;
    const int swz = (lrow >> 1) & (CH - 1);
    unsigned offa[KS], offb[KS];
#pragma unroll
    for (int s = 0; s < KS; s++) {
        const int chunk = 4 * (kg * KS + s) + lgrp;
        offa[s] = (wm * WTM + lrow) * BK + ((chunk ^ swz) << 4);
        offb[s] = SIZE_A + (wn * WTN + lrow) * BK + ((chunk ^ swz) << 4);
    }

    v4i acc[NBM][NBN];
#pragma unroll
    for (int i = 0; i < NBM; i++)
#pragma unroll
        for (int j = 0; j < NBN; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[i][j][v] = 0;

    // Two register slots of a K tile's fragments: fa[slot][s*NBM + i], fb[slot][s*NBN + j].
    v4i fa[2][NFA], fb[2][NFB];
    auto read_frag = [&](unsigned base, auto S, auto F) {
        constexpr int sl = decltype(S)::value, f = decltype(F)::value;
        if constexpr (f < NFA) lds_read16<(f % NBM) * 16 * BK>(fa[sl][f], base + offa[f / NBM]);
        else lds_read16<((f - NFA) % NBN) * 16 * BK>(fb[sl][f - NFA], base + offb[(f - NFA) / NBN]);
    };
    auto land = [&](auto S) {  // the slot's reads have retired: fence, re-centre A
        constexpr int sl = decltype(S)::value;
        lds_wait<0>();
        static_for<0, NFA>([&](auto F) { reg_fence(fa[sl][F.value]); });
        static_for<0, NFB>([&](auto F) { reg_fence(fb[sl][F.value]); });
        static_for<0, NFA>([&](auto F) { fa[sl][F.value] ^= (int)0x80808080u; });
    };

    __builtin_amdgcn_s_barrier();  // P0
    static_for<0, NF>([&](auto F) { read_frag(lds0, IC<0>{}, F); });
    land(IC<0>{});

    // One K tile from slot S: MFMA 0, the barrier, then the next tile's NF
    // reads spread over the gaps of the first half of the tile's MFMAs; the
    // next slot lands before the last MFMA.
    auto tile = [&](int kt, auto S) {
        constexpr int sl = decltype(S)::value, ns = 1 - sl;
        const unsigned nbase = lds0 + ((kt + 1) % STAGES) * STAGE;
        constexpr int RPG = (NF + NM / 2 - 1) / (NM / 2);  // reads per gap
        static_for<0, NM>([&](auto Q) {
            constexpr int q = Q.value;
            constexpr int s = q / (NBM * NBN), j = (q / NBM) % NBN, i = q % NBM;
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[sl][s * NBM + i], fb[sl][s * NBN + j],
                                                              acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (q == 0) __builtin_amdgcn_s_barrier();  // B(kt)
            if constexpr (q < NM / 2)
                static_for<q * RPG, (q + 1) * RPG < NF ? (q + 1) * RPG : NF>(
                    [&](auto F) { read_frag(nbase, IC<ns>{}, F); });
            if constexpr (q == NM - 2) land(IC<ns>{});
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    // Tiles in pairs (the slot index is a compile-time constant). The last
    // tile's reads ahead are issued too, without a branch: they read the
    // stage after it, inside the ring and no longer written by any DMA (the
    // producers waited for every tile before its barrier), and are unused.
    for (int kt = 0; kt < nk; kt += 2) {
        tile(kt, IC<0>{});
        if (kt + 1 < nk) tile(kt + 1, IC<1>{});
    }
    lds_wait<0>();

    // Stores. A 16x16 block puts 4 rows x 16 columns in a register (64-byte
    // row pieces per store); blocks j and j+1 are regrouped with two lane
    // swaps so each store writes 2 rows x 32 columns (whole 128-byte lines):
    // with X = block j, Y = block j+1 and row groups g = lane/16,
    // permlane16_swap gives X = [X0 Y0 X2 Y2], Y = [X1 Y1 X3 Y3], then
    // permlane32_swap X = [X0 Y0 X1 Y1] (rows r, 4+r), Y = [X2 Y2 X3 Y3]
    // (rows 8+r, 12+r). Row blocks RB0 .. RB0+NRB-1 of the wave tile.
    auto store_rows = [&](auto RB0, auto NRB, auto CHECK) {
        constexpr int rb0 = decltype(RB0)::value, nrb = decltype(NRB)::value;
        constexpr bool chk = decltype(CHECK)::value != 0;
        const int hrow = 4 * (lane >> 5), hcol = lane & 31;
        static_for<0, nrb>([&](auto I) {
            constexpr int i = rb0 + I.value;
            static_for<0, 4>([&](auto V) {
                constexpr int v = V.value;
                const float rs = sav[I.value * 4 + v];
                static_for<0, NBN / 2>([&](auto JP) {
                    constexpr int j0 = 2 * JP.value;
                    unsigned x, y;
                    if constexpr (OUT == 0) {
                        x = (unsigned)acc[i][j0][v];
                        y = (unsigned)acc[i][j0 + 1][v];
                    } else {
                        const float dx = (OUT == 2) ? rs * sbv[j0] : sbv[j0];
                        const float dy = (OUT == 2) ? rs * sbv[j0 + 1] : sbv[j0 + 1];
                        x = __float_as_uint((float)(int32_t)((unsigned)acc[i][j0][v] + offv[j0]) * dx);
                        y = __float_as_uint((float)(int32_t)((unsigned)acc[i][j0 + 1][v] + offv[j0 + 1]) * dy);
                    }
                    const auto p16 = __builtin_amdgcn_permlane16_swap(x, y, false, false);
                    const auto p32 = __builtin_amdgcn_permlane32_swap(p16[0], p16[1], false, false);
                    const int col = wcol0 + j0 * 16 + hcol;
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const int row = wrow0 + i * 16 + 8 * h + hrow + v;
                        if (chk && (row >= Mv || col >= Nv)) continue;
                        const long o = (long)row * ld_out + col;
                        const unsigned val = h == 0 ? p32[0] : p32[1];
                        if constexpr (NTS) __builtin_nontemporal_store(val, (gu32_t *)C_out + o);
                        else ((gu32_t *)C_out)[o] = val;
                    }
                });
            });
        });
    };
    const bool inside = m0 + BM <= Mv && n0 + BN <= Nv;
    if constexpr (KGR == 1) {
        if (inside) store_rows(IC<0>{}, IC<NBM>{}, IC<0>{});
        else store_rows(IC<0>{}, IC<NBM>{}, IC<1>{});
    } else {
        // Partial-tile exchange: group kg stores the 32 rows of its wave tile
        // it does not own lane-linearly into its 8 KB of the freed ring; after
        // the barrier it adds its partner's copy of its own half (the partner
        // is wave ^ 4), then stores that half.
        constexpr int HB = NBM / 2;
        auto exchange_and_store = [&](auto KG) {
            constexpr int own = decltype(KG)::value, oth = 1 - own;
            const unsigned waddr = lds0 + wave * XW + lane * 16, paddr = lds0 + (wave ^ 4) * XW + lane * 16;
            static_for<0, HB * NBN>([&](auto P) {
                constexpr int i = oth * HB + P.value / NBN, j = P.value % NBN;
                lds_write16<P.value * 1024>(waddr, acc[i][j]);
            });
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();  // exchange
            v4i t[HB * NBN];
            static_for<0, HB * NBN>([&](auto P) { lds_read16<P.value * 1024>(t[P.value], paddr); });
            lds_wait<0>();
            static_for<0, HB * NBN>([&](auto P) {
                constexpr int i = own * HB + P.value / NBN, j = P.value % NBN;
                reg_fence(t[P.value]);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[i][j][e] = (int)((unsigned)acc[i][j][e] + (unsigned)t[P.value][e]);
            });
            if (inside) store_rows(IC<own * HB>{}, IC<HB>{}, IC<0>{});
            else store_rows(IC<own * HB>{}, IC<HB>{}, IC<1>{});
        };
        if (kg == 0) exchange_and_store(IC<0>{});
        else exchange_and_store(IC<1>{});
    }
}

// ---------------------------------------------------------------------------
// Persistent form of igemm_kg_kernel for grids of many 128x128 tiles (the
// 50257-vocab head): the consumers of igemm_kg_kernel (one K group, eight
// waves of 32x64 on v_mfma_i32_16x16x64_i8, a whole K tile's fragments read
// one tile ahead) and the producers of igemm_wp_kernel (the K-tile stream runs
// across output tiles through the ring; the epilogue operands of a tile are
// DMA'd into LDS, three tiles deep, so the consumers never wait on vmcnt and
// the stores of one tile drain under the next). Row classes as in
// igemm_wp_kernel (P, col_shift). K is a multiple of 256 (an even number of
// K tiles per output tile: the two fragment slots alternate within a tile and
// the reads ahead of a tile's last K tile are the next tile's first).
//
// DYN: tiles handed out from a counter per XCD instead of fixed slots, so a
// workgroup that starts late (its CU busy) takes fewer tiles and no tile
// waits for it. The workgroups of XCD x (blockIdx % 8 == x) share the
// logical tiles i * grid + s0 + j (its slots s0 .. s0 + cnt - 1, every round
// i) in that order: elements j and cnt + j are workgroup j's first two
// tiles (as with fixed slots), element 2 cnt + v goes to the fetch that
// returns v from tile_ctr[x]. One more wave (the scheduler, no DMA, no MFMA)
// fetches tile t + 2 when tile t starts (one atomic add with return, lane
// 0), until a fetch has come back past the list, and at tile t's last K tile
// -- a tile later, the atomic's latency covered; atomics are its only memory
// operations, so neither the DMA stream nor the output stores wait behind
// one -- writes the tile's logical index (or -1) into an LDS ring of four
// before that K tile's barrier. The producers read it two barriers later, at
// least STAGES K tiles before its first DMA (nk >= STAGES + 1), the consumers
// at the end of tile t + 1; every wave sees the same sequence of tiles and
// runs the same barriers. When its fetches are done every workgroup adds one
// to tile_ctr[8 + x]; the last of the XCD's workgroups resets both counters
// for the next launch (stream order). Counters start at zero.
template <int STAGES, int NWP, int OUT, int NTS, int DYN>
__global__ __launch_bounds__(64 * (8 + NWP + DYN)) __attribute__((amdgpu_waves_per_eu(
    (8 + NWP + DYN + 3) / 4))) void igemm_kgp_kernel(const uint8_t *__restrict__ A, long lda,
                                              const int8_t *__restrict__ B, long ldb,
                                              const int32_t *__restrict__ col_off,
                                              const float *__restrict__ sa,
                                              const float *__restrict__ sb,
                                              void *__restrict__ Cv, long ldc, int M, int N, int K,
                                              int P, int col_shift, int gm, int *__restrict__ tile_ctr) {
    constexpr int BM = 128, BN = 128, BK = IG_BK, CH = BK / 16, RPI = 1024 / BK;
    constexpr int SIZE_A = BM * BK, STAGE = (BM + BN) * BK;
    constexpr int PIA = BM / (RPI * NWP), PIB = BN / (RPI * NWP), PL = PIA + PIB;
    constexpr int SCL = 2 * BN + BM + 128;      // floats per tile: sb, col_off, sa, spare
    constexpr int NS = OUT != 0 ? 8 / NWP : 0;  // epilogue-operand DMA instructions per producer
    constexpr int LDS_BYTES = STAGES * STAGE + 3 * SCL * 4 + 16;
    static_assert(NWP == 2 || NWP == 4, "producer waves");
    static_assert(STAGES >= 3 && LDS_BYTES <= 160 * 1024, "ring");
    static_assert((STAGES - 1) * (PL + NS) <= 63, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) int8_t lds[LDS_BYTES];
    float *scl = reinterpret_cast<float *>(lds + STAGES * STAGE);  // [3 tiles][sb | col_off | sa]
    int *ring = reinterpret_cast<int *>(lds + STAGES * STAGE + 3 * SCL * 4);  // DYN: later tiles

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int Mc = (M + P - 1) / P;
    const int nbm = P * ((Mc + BM - 1) / BM), nbn = (N + (col_shift ? 31 : 0) + BN - 1) / BN;
    const int ntiles = nbm * nbn;
    const int cb0 = col_shift ? (int)((reinterpret_cast<unsigned long>(Cv) >> 2) & 31) : 0;
    const int nb = gridDim.x;
    const int slot = xcd_remap(blockIdx.x, nb);
    const int my_tiles = slot < ntiles ? (ntiles - 1 - slot) / nb + 1 : 0;
    const int nk = K / BK;
    // K tiles this workgroup streams: all of them known here, or (DYN) the
    // first AH + 1 tiles', growing as later ones are handed out
    constexpr int AH = 1;  // DYN: tiles by slot beyond the first
    int G = DYN ? min(my_tiles, AH + 1) * nk : my_tiles * nk;
    if (G == 0) return;  // uniform: no barrier is left unmatched
    // DYN: this XCD's slots s0 .. s0 + cnt - 1 and how many of its logical
    // tiles exist (valid_x): element k of its list is tile
    // (k / cnt) * nb + s0 + k % cnt, increasing in k
    const int xcd = blockIdx.x % 8, xq = nb / 8, xr = nb % 8;
    const int s0 = xcd * xq + min(xcd, xr), cnt = xq + (xcd < xr ? 1 : 0);
    const int valid_x = (ntiles / nb) * cnt + min(max(ntiles % nb - s0, 0), cnt);
    auto tile_origin = [&](int logical, int &cls, int &r0, int &n0) {
        int bm, bn;
        tile_coords(logical, nbm, nbn, gm, bm, bn);
        cls = bm % P;
        r0 = bm / P * BM;
        n0 = bn * BN - (col_shift ? (int)((cb0 + (long)cls * ldc) & 31) : 0);
    };
    // logical tile of local tile i (fixed slots; DYN: the first AH + 1 by
    // slot, later ones from the ring)
    auto logical_of = [&](int i) {
        return DYN && i > AH ? __builtin_amdgcn_readfirstlane(ring[i & 3]) : i * nb + slot;
    };

    if (DYN && wave == 8 + NWP) {
        // ------------------------------------------------------ scheduler
        static_assert(AH == 1, "one fetch in flight, made and used within a tile");
        int Gs = G;
        bool more = my_tiles >= AH + 1;  // tile t + 1 exists and no fetch came back empty
        __builtin_amdgcn_s_barrier();    // P0
        for (int t = 0; t * nk < Gs; t++) {
            // Tile t starts: fetch tile t + 2. The atomic runs on lane 0
            // alone (exec narrowed inside the asm) and every tile, adding 0
            // once fetching is over: its result register is then defined on
            // every path and read only after the wait below (the compiler,
            // unaware of the atomic, would otherwise copy it at a merge
            // before it lands; its own atomic would wait for it at once).
            int fetched;
            unsigned long long exec_save;
            const int inc = more ? 1 : 0, voff0 = 0;
            asm volatile(
                "s_mov_b64 %1, exec\n\t"
                "s_mov_b64 exec, 1\n\t"
                "global_atomic_add %0, %2, %3, %4 sc0\n\t"
                "s_mov_b64 exec, %1"
                : "=&v"(fetched), "=&s"(exec_save)
                : "v"(voff0), "v"(inc), "s"(tile_ctr + xcd)
                : "memory");
            for (int kk = 0; kk < nk; kk++) {
                if (kk == nk - 1 && inc) {
                    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
                    asm volatile("" : "+v"(fetched));
                    const int v = __builtin_amdgcn_readfirstlane(fetched);
                    const int k = (AH + 1) * cnt + v;
                    const int nxt = k < valid_x ? (k / cnt) * nb + s0 + k % cnt : -1;
                    if (lane == 0) ring[(t + AH + 1) & 3] = nxt;
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    if (nxt >= 0) Gs += nk;
                    else more = false;
                }
                __builtin_amdgcn_s_barrier();  // B(t nk + kk)
            }
        }
        // every fetch of this workgroup has returned: count it done; the
        // XCD's last workgroup resets its counters
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        if (lane == 0 && atomicAdd(tile_ctr + IGEMM_TILE_CTRS / 2 + xcd, 1) == cnt - 1) {
            atomicExch(tile_ctr + xcd, 0);
            atomicExch(tile_ctr + IGEMM_TILE_CTRS / 2 + xcd, 0);
        }
        return;
    }

    if (wave >= 8) {
        // ------------------------------------------------------ producers
        const int pw = wave - 8;
        const int8_t *A8 = reinterpret_cast<const int8_t *>(A);
        unsigned voff[PL];
        int ldso[PL];
        // Output tile i starts: its rows' and columns' source offsets, and the
        // 4-byte DMA of its epilogue operands into LDS buffer i % 3 (pieces as
        // in igemm_wp_kernel: sb 0-1, col_off 2-3, sa 4-5, absent ones load
        // sb again into the spare slot).
        auto begin_tile = [&](int i) {
            int cls, r0, n0;
            tile_origin(logical_of(i), cls, r0, n0);
#pragma unroll
            for (int d = 0; d < PL; d++) {
                const bool isA = d < PIA;
                const int rb = ((isA ? d : d - PIA) * NWP + pw) * RPI;
                const int r = rb + lane / CH;
                const int c = (lane % CH) ^ ((r >> 1) & (CH - 1));
                const int grow = isA ? min(cls + P * (r0 + r), M - 1) : max(min(n0 + r, N - 1), 0);
                voff[d] = (unsigned)grow * (unsigned)(isA ? lda : ldb) + (unsigned)(c * 16);
                ldso[d] = (isA ? 0 : SIZE_A) + rb * BK;
            }
            if (OUT != 0) {
                float *dst = scl + (i % 3) * SCL;
#pragma unroll
                for (int h = 0; h < NS; h++) {
                    const int piece = pw * NS + h;
                    const float *src = sb + max(min(n0 + (piece & 1) * 64 + lane, N - 1), 0);
                    float *to = dst + 2 * BN + BM + (piece & 1) * 64;  // spare slot
                    if (piece < 2) {
                        to = dst + piece * 64;
                    } else if (piece < 4) {
                        if (col_off) {
                            src = reinterpret_cast<const float *>(col_off) +
                                  max(min(n0 + (piece - 2) * 64 + lane, N - 1), 0);
                            to = dst + BN + (piece - 2) * 64;
                        }
                    } else if (OUT == 2 && piece < 6) {
                        src = sa + min(cls + P * (r0 + (piece - 4) * 64 + lane), M - 1);
                        to = dst + 2 * BN + (piece - 4) * 64;
                    }
                    __builtin_amdgcn_global_load_lds((const void *)src, (lds_void_t *)to, 4, 0, 0);
                }
            }
        };
        int di = 0, dk = 0;  // output tile and K tile of the next DMA
        auto dma_next = [&]() -> bool {
            const bool first = dk == 0;
            if (first) begin_tile(di);
            const long koff = (long)dk * BK;
            int8_t *stage = lds + ((di * nk + dk) % STAGES) * STAGE;
#pragma unroll
            for (int d = 0; d < PL; d++)
                __builtin_amdgcn_global_load_lds((const void *)((d < PIA ? A8 : B) + koff + voff[d]),
                                                 (lds_void_t *)(stage + ldso[d]), 16, 0, 0);
            if (++dk == nk) {
                dk = 0;
                di++;
            }
            return first && NS > 0;
        };
        // hist bit j: the j-th most recently issued K-tile DMA carried
        // epilogue operands (NS more vmcnt entries, issued before its PL).
        unsigned hist = 0;
        auto wait_younger = [&](auto NYC) {  // the NY youngest K tiles may still fly
            constexpr int ny = decltype(NYC)::value;
            const int c = __builtin_popcount(hist & ((1u << ny) - 1));
            static_for<0, ny + 1>([&](auto Cc) {
                constexpr int cc = decltype(Cc)::value;
                if (c == cc) __builtin_amdgcn_s_waitcnt(waitcnt_vm(ny * PL + cc * NS));
            });
        };
        // Prologue as in igemm_kg_kernel: K tiles 0 and 1, P0 once tile 0 has
        // landed, then the rest of the ring.
        hist = (hist << 1) | (dma_next() ? 1u : 0u);
        if (G > 1) {
            hist = (hist << 1) | (dma_next() ? 1u : 0u);
            wait_younger(IC<1>{});
        } else {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        }
        __builtin_amdgcn_s_barrier();  // P0
#pragma unroll
        for (int t = 2; t < STAGES; t++)
            if (t < G) hist = (hist << 1) | (dma_next() ? 1u : 0u);
        for (int g = 0; g < G; g++) {
            // DYN: tile t > AH was published before B((t - 1) nk - 1); read
            // it here, STAGES or more K tiles before its first DMA
            if (DYN && g >= AH * nk + 1 && g % nk == 1 &&
                __builtin_amdgcn_readfirstlane(ring[(g / nk + 1) & 3]) >= 0)
                G += nk;
            // K tile g+1 has landed; tiles g+2 .. g+STAGES-1 may still fly
            if (g + STAGES - 1 < G) wait_younger(IC<STAGES - 2>{});
            else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            __builtin_amdgcn_s_barrier();  // B(g)
            if (g + STAGES < G) hist = (hist << 1) | (dma_next() ? 1u : 0u);
        }
        return;
    }

    // ---------------------------------------------------------- consumers
    constexpr int WTM = 32, WTN = 64;           // wave tile (4 x 2 waves)
    constexpr int NBM = WTM / 16, NBN = WTN / 16;  // 16x16 blocks
    constexpr int KS = 2;                       // 64-byte k-steps per K tile
    constexpr int NFA = KS * NBM, NFB = KS * NBN, NF = NFA + NFB;
    constexpr int NM = KS * NBM * NBN;          // MFMAs per K tile
    const int wm = wave >> 1, wn = wave & 1;
    void *C_out = Cv;
    long ld_out = ldc;
    int Mv = M, Nv = N, Pv = P;
    asm volatile("" : "+s"(C_out), "+s"(ld_out), "+s"(Mv), "+s"(Nv), "+s"(Pv));
    const int lcol = lane & 15;
    const unsigned lds0 = lds_addr(lds);
    const int lrow = lane & 15, lgrp = lane >> 4;
    const int swz = (lrow >> 1) & (CH - 1);
    unsigned offa[KS], offb[KS];
#pragma unroll
    for (int s = 0; s < KS; s++) {
        const int chunk = 4 * s + lgrp;
        offa[s] = (wm * WTM + lrow) * BK + ((chunk ^ swz) << 4);
        offb[s] = SIZE_A + (wn * WTN + lrow) * BK + ((chunk ^ swz) << 4);
    }

    v4i acc[NBM][NBN];
#pragma unroll
    for (int i = 0; i < NBM; i++)
#pragma unroll
        for (int j = 0; j < NBN; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[i][j][v] = 0;

    v4i fa[2][NFA], fb[2][NFB];
    auto read_frag = [&](unsigned base, auto S, auto F) {
        constexpr int sl = decltype(S)::value, f = decltype(F)::value;
        if constexpr (f < NFA) lds_read16<(f % NBM) * 16 * BK>(fa[sl][f], base + offa[f / NBM]);
        else lds_read16<((f - NFA) % NBN) * 16 * BK>(fb[sl][f - NFA], base + offb[(f - NFA) / NBN]);
    };
    auto land = [&](auto S) {
        constexpr int sl = decltype(S)::value;
        lds_wait<0>();
        static_for<0, NFA>([&](auto F) { reg_fence(fa[sl][F.value]); });
        static_for<0, NFB>([&](auto F) { reg_fence(fb[sl][F.value]); });
        static_for<0, NFA>([&](auto F) { fa[sl][F.value] ^= (int)0x80808080u; });
    };

    __builtin_amdgcn_s_barrier();  // P0
    static_for<0, NF>([&](auto F) { read_frag(lds0, IC<0>{}, F); });
    land(IC<0>{});

    // K tile g (global index in this workgroup's stream) from slot S: MFMA 0,
    // the barrier, the next K tile's reads over the first half of the MFMAs,
    // the next slot landed before the last MFMA. The reads ahead of the last
    // K tile of the stream read a stage inside the ring that no DMA writes
    // any more, and are unused.
    auto ktile = [&](int g, auto S) {
        constexpr int sl = decltype(S)::value, ns = 1 - sl;
        const unsigned nbase = lds0 + ((g + 1) % STAGES) * STAGE;
        constexpr int RPG = (NF + NM / 2 - 1) / (NM / 2);
        static_for<0, NM>([&](auto Q) {
            constexpr int q = Q.value;
            constexpr int s = q / (NBM * NBN), j = (q / NBM) % NBN, i = q % NBM;
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[sl][s * NBM + i], fb[sl][s * NBN + j],
                                                              acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (q == 0) __builtin_amdgcn_s_barrier();  // B(g)
            if constexpr (q < NM / 2)
                static_for<q * RPG, (q + 1) * RPG < NF ? (q + 1) * RPG : NF>(
                    [&](auto F) { read_frag(nbase, IC<ns>{}, F); });
            if constexpr (q == NM - 2) land(IC<ns>{});
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    int g = 0;
    for (int t = 0; DYN || t < my_tiles; t++) {
        for (int kt = 0; kt < nk; kt += 2, g += 2) {
            ktile(g, IC<0>{});
            ktile(g + 1, IC<1>{});
        }
        // DYN: tile t + 1 (the first AH + 1 by slot; later ones published
        // before B(t nk - 1), read after this tile's last barrier)
        const int next = !DYN ? 0 : t + 1 <= AH ? (my_tiles >= t + 2 ? 1 : -1)
                                                : __builtin_amdgcn_readfirstlane(ring[(t + 1) & 3]);
        // Epilogue of tile t (operands from LDS buffer t % 3; stores as in
        // igemm_kg_kernel, 2 rows x 32 columns per store after two lane
        // swaps). The stores carry no wait: they drain under tile t + 1.
        int cls, r0, n0;
        tile_origin(logical_of(t), cls, r0, n0);
        const float *sc = scl + (t % 3) * SCL;
        const int wrow0 = r0 + wm * WTM, wcol0 = n0 + wn * WTN;  // class-local row
        float sbv[NBN], sav[8];
        unsigned offv[NBN];
#pragma unroll
        for (int j = 0; j < NBN; j++) {
            const int cl = wn * WTN + j * 16 + lcol;
            sbv[j] = (OUT != 0) ? sc[cl] : 0.f;
            offv[j] = (OUT != 0 && col_off) ? reinterpret_cast<const unsigned *>(sc)[BN + cl] : 0u;
        }
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int r = (q >> 2) * 16 + 4 * (lane >> 4) + (q & 3);
            sav[q] = (OUT == 2) ? sc[2 * BN + wm * WTM + r] : 0.f;
        }
        auto store_rows = [&](auto CHECK) {
            constexpr bool chk = decltype(CHECK)::value != 0;
            const int hrow = 4 * (lane >> 5), hcol = lane & 31;
            static_for<0, NBM>([&](auto I) {
                constexpr int i = I.value;
                static_for<0, 4>([&](auto V) {
                    constexpr int v = V.value;
                    const float rs = sav[i * 4 + v];
                    static_for<0, NBN / 2>([&](auto JP) {
                        constexpr int j0 = 2 * JP.value;
                        unsigned x, y;
                        if constexpr (OUT == 0) {
                            x = (unsigned)acc[i][j0][v];
                            y = (unsigned)acc[i][j0 + 1][v];
                        } else {
                            const float dx = (OUT == 2) ? rs * sbv[j0] : sbv[j0];
                            const float dy = (OUT == 2) ? rs * sbv[j0 + 1] : sbv[j0 + 1];
                            x = __float_as_uint((float)(int32_t)((unsigned)acc[i][j0][v] + offv[j0]) * dx);
                            y = __float_as_uint((float)(int32_t)((unsigned)acc[i][j0 + 1][v] + offv[j0 + 1]) * dy);
                        }
                        const auto p16 = __builtin_amdgcn_permlane16_swap(x, y, false, false);
                        const auto p32 = __builtin_amdgcn_permlane32_swap(p16[0], p16[1], false, false);
                        const int col = wcol0 + j0 * 16 + hcol;
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            const int row = cls + Pv * (wrow0 + i * 16 + 8 * h + hrow + v);
                            if (chk && (row >= Mv || col < 0 || col >= Nv)) continue;
                            const long o = (long)row * ld_out + col;
                            const unsigned val = h == 0 ? p32[0] : p32[1];
                            if constexpr (NTS) __builtin_nontemporal_store(val, (gu32_t *)C_out + o);
                            else ((gu32_t *)C_out)[o] = val;
                        }
                    });
                });
            });
        };
        if (cls + Pv * (r0 + BM - 1) < Mv && n0 >= 0 && n0 + BN <= Nv) store_rows(IC<0>{});
        else store_rows(IC<1>{});
#pragma unroll
        for (int i = 0; i < NBM; i++)
#pragma unroll
            for (int j = 0; j < NBN; j++)
#pragma unroll
                for (int v = 0; v < 4; v++) acc[i][j][v] = 0;
        if (DYN && next < 0) break;
    }
    lds_wait<0>();
}

static int device_cus() {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    return cus;
}

// Row classes of a 4-byte output (igemm_wp_kernel): rows r and r + P start at
// the same offset within a 128-byte line; shift: some row starts off a line.
struct RowClasses {
    int P, shift;
};
static RowClasses row_classes(const void *C, long ldc) {
    const int lm = (int)(ldc & 31), cb = (int)((reinterpret_cast<uintptr_t>(C) >> 2) & 31);
    return RowClasses{lm ? 32 / (lm & -lm) : 1, (lm || cb) ? 1 : 0};
}
// Whether the row-class tiling suits an output: its rows are off lines and
// the classes fill BM-row tiles with at most 1/8 of the tile rows idle.
static bool classes_fill(int M, long ldc, const void *C, int BM) {
    const RowClasses rc = row_classes(C, ldc);
    if (!rc.shift || M <= 0) return false;
    const long Mc = (M + rc.P - 1) / rc.P;
    return (long)rc.P * ((Mc + BM - 1) / BM * BM) * 8 <= (long)M * 9;
}

template <int BM, int BN, int WM, int WN, int STAGES, int NWP>
static hipError_t launch_wp_band(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                                 const int8_t *B, long ldb, const int32_t *col_off,
                                 const float *sa, const float *sb, void *C, long ldc, bool classes,
                                 hipStream_t stream) {
    const RowClasses rc = classes ? row_classes(C, ldc) : RowClasses{1, 0};
    const int gm = rc.P > 1 ? 16 : 8;  // 16 classes x 2 column tiles per XCD and round
    const long Mc = (M + rc.P - 1) / rc.P;
    const long ntiles = rc.P * ((Mc + BM - 1) / BM) * ((N + (rc.shift ? 31 : 0) + BN - 1) / BN);
    if (M == 0 || N == 0 || K / IG_BK == 0) return hipSuccess;
    const int grid = (int)(ntiles < device_cus() ? ntiles : device_cus());
    const dim3 block(64 * (WM * WN + NWP));
    // streaming (non-temporal) stores at every size: on the 823 MB output of
    // the 50257-vocab head they take 386-392 us against 425-436 us for plain
    // stores (two boxes, same build). The hint is a compile-time choice (a
    // run-time choice between two otherwise equal stores is merged by the
    // compiler into one without it).
    auto go = [&](auto NT) {
        constexpr int nts = decltype(NT)::value;
        switch (out_mode) {
            case 0:
                hipLaunchKernelGGL((igemm_wp_kernel<BM, BN, WM, WN, STAGES, NWP, 0, nts>), dim3(grid), block, 0,
                                   stream, A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K, rc.P, rc.shift, gm);
                break;
            case 1:
                hipLaunchKernelGGL((igemm_wp_kernel<BM, BN, WM, WN, STAGES, NWP, 1, nts>), dim3(grid), block, 0,
                                   stream, A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K, rc.P, rc.shift, gm);
                break;
            default:
                hipLaunchKernelGGL((igemm_wp_kernel<BM, BN, WM, WN, STAGES, NWP, 2, nts>), dim3(grid), block, 0,
                                   stream, A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K, rc.P, rc.shift, gm);
                break;
        }
    };
    go(IC<1>{});
    return hipGetLastError();
}

// 32-bit per-lane DMA offsets: row bands of A and column bands of B whose
// byte spans stay below 2^31 (as launch_split does for igemm_mfma_kernel).
template <int BM, int BN, int WM, int WN, int STAGES, int NWP = 4>
static hipError_t launch_wp(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                            const int8_t *B, long ldb, const int32_t *col_off, const float *sa,
                            const float *sb, void *C, long ldc, bool classes, hipStream_t stream) {
    const long LIM = 1L << 31;
    long mband = lda > 0 ? LIM / lda : M, nband = ldb > 0 ? LIM / ldb : N;
    mband = mband >= M ? M : (mband / BM) * BM;
    nband = nband >= N ? N : (nband / BN) * BN;
    if (mband <= 0 || nband <= 0) return hipErrorInvalidValue;
    for (long m = 0; m < M; m += mband) {
        for (long n = 0; n < N; n += nband) {
            const int mm = (int)(M - m < mband ? M - m : mband);
            const int nn = (int)(N - n < nband ? N - n : nband);
            hipError_t e = launch_wp_band<BM, BN, WM, WN, STAGES, NWP>(
                out_mode, mm, nn, K, A + m * lda, lda, B + n * ldb, ldb,
                col_off ? col_off + n : nullptr, sa ? sa + m : nullptr, sb ? sb + n : nullptr,
                (char *)C + (m * ldc + n) * 4, ldc, classes, stream);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

// The persistent 16x16x64 kernel over 128x128 tiles (row classes optional).
// tile_ctr (IGEMM_TILE_CTRS zeroed ints, or NULL): tiles handed out per XCD
// from these counters when a tile has more than STAGES K tiles, else fixed
// slots.
template <int STAGES, int NWP>
static hipError_t launch_kgp_band(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                                  const int8_t *B, long ldb, const int32_t *col_off, const float *sa,
                                  const float *sb, void *C, long ldc, bool classes, int *tile_ctr,
                                  hipStream_t stream) {
    if (M == 0 || N == 0 || K / IG_BK == 0) return hipSuccess;
    if (K % (2 * IG_BK) != 0) return hipErrorInvalidValue;  // an even number of K tiles
    const RowClasses rc = classes ? row_classes(C, ldc) : RowClasses{1, 0};
    const int gm = rc.P > 1 ? 16 : 8;
    const long Mc = (M + rc.P - 1) / rc.P;
    const long ntiles = rc.P * ((Mc + 127) / 128) * ((N + (rc.shift ? 31 : 0) + 127) / 128);
    const int grid = (int)(ntiles < device_cus() ? ntiles : device_cus());
    const bool dyn = tile_ctr != nullptr && K / IG_BK >= STAGES + 1;
    const dim3 block(64 * (8 + NWP + (dyn ? 1 : 0)));
    auto go = [&](auto OUTC, auto DYNC) {
        constexpr int o = decltype(OUTC)::value, dy = decltype(DYNC)::value;
        hipLaunchKernelGGL((igemm_kgp_kernel<STAGES, NWP, o, 1, dy>), dim3(grid), block, 0, stream, A, lda, B,
                           ldb, col_off, sa, sb, C, ldc, M, N, K, rc.P, rc.shift, gm, dy ? tile_ctr : nullptr);
    };
    auto go_out = [&](auto DYNC) {
        switch (out_mode) {
            case 0: go(IC<0>{}, DYNC); break;
            case 1: go(IC<1>{}, DYNC); break;
            default: go(IC<2>{}, DYNC); break;
        }
    };
    if (dyn) go_out(IC<1>{});
    else go_out(IC<0>{});
    return hipGetLastError();
}

// 32-bit per-lane DMA offsets: row bands of A and column bands of B whose
// byte spans stay below 2^31.
template <int STAGES, int NWP>
static hipError_t launch_kgp(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                             const int8_t *B, long ldb, const int32_t *col_off, const float *sa,
                             const float *sb, void *C, long ldc, bool classes, int *tile_ctr,
                             hipStream_t stream) {
    const long LIM = 1L << 31;
    long mband = lda > 0 ? LIM / lda : M, nband = ldb > 0 ? LIM / ldb : N;
    mband = mband >= M ? M : (mband / 128) * 128;
    nband = nband >= N ? N : (nband / 128) * 128;
    if (mband <= 0 || nband <= 0) return hipErrorInvalidValue;
    for (long m = 0; m < M; m += mband) {
        for (long n = 0; n < N; n += nband) {
            const int mm = (int)(M - m < mband ? M - m : mband);
            const int nn = (int)(N - n < nband ? N - n : nband);
            hipError_t e = launch_kgp_band<STAGES, NWP>(
                out_mode, mm, nn, K, A + m * lda, lda, B + n * ldb, ldb, col_off ? col_off + n : nullptr,
                sa ? sa + m : nullptr, sb ? sb + n : nullptr, (char *)C + (m * ldc + n) * 4, ldc, classes,
                tile_ctr, stream);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

template <int STAGES, int NWP, int KGR>
static hipError_t launch_kg_band(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                                 const int8_t *B, long ldb, const int32_t *col_off,
                                 const float *sa, const float *sb, void *C, long ldc,
                                 hipStream_t stream) {
    const int nblk = ((M + 127) / 128) * ((N + 127) / 128);
    if (nblk == 0 || K / IG_BK == 0) return hipSuccess;
    const dim3 grid(nblk), block(64 * (8 + NWP));
    const bool nt = (long)M * N * 4 <= (256L << 20);  // outputs up to 256 MiB: streaming stores
    auto go = [&](auto NT) {
        constexpr int nts = decltype(NT)::value;
        switch (out_mode) {
            case 0:
                hipLaunchKernelGGL((igemm_kg_kernel<STAGES, NWP, KGR, 0, nts>), grid, block, 0, stream, A, lda, B,
                                   ldb, col_off, sa, sb, C, ldc, M, N, K);
                break;
            case 1:
                hipLaunchKernelGGL((igemm_kg_kernel<STAGES, NWP, KGR, 1, nts>), grid, block, 0, stream, A, lda, B,
                                   ldb, col_off, sa, sb, C, ldc, M, N, K);
                break;
            default:
                hipLaunchKernelGGL((igemm_kg_kernel<STAGES, NWP, KGR, 2, nts>), grid, block, 0, stream, A, lda, B,
                                   ldb, col_off, sa, sb, C, ldc, M, N, K);
                break;
        }
    };
    if (nt) go(IC<1>{});
    else go(IC<0>{});
    return hipGetLastError();
}

// 32-bit per-lane DMA offsets: row bands of A and column bands of B whose
// byte spans stay below 2^31 (as launch_split).
template <int STAGES, int NWP, int KGR>
static hipError_t launch_kg(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                            const int8_t *B, long ldb, const int32_t *col_off, const float *sa,
                            const float *sb, void *C, long ldc, hipStream_t stream) {
    const long LIM = 1L << 31;
    long mband = lda > 0 ? LIM / lda : M, nband = ldb > 0 ? LIM / ldb : N;
    mband = mband >= M ? M : (mband / 128) * 128;
    nband = nband >= N ? N : (nband / 128) * 128;
    if (mband <= 0 || nband <= 0) return hipErrorInvalidValue;
    for (long m = 0; m < M; m += mband) {
        for (long n = 0; n < N; n += nband) {
            const int mm = (int)(M - m < mband ? M - m : mband);
            const int nn = (int)(N - n < nband ? N - n : nband);
            hipError_t e = launch_kg_band<STAGES, NWP, KGR>(
                out_mode, mm, nn, K, A + m * lda, lda, B + n * ldb, ldb, col_off ? col_off + n : nullptr,
                sa ? sa + m : nullptr, sb ? sb + n : nullptr, (char *)C + (m * ldc + n) * 4, ldc, stream);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

template <int BM, int BN, int WM, int WN, int STAGES, int OCC>
static hipError_t launch_icfg(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                              const int8_t *B, long ldb, const int32_t *col_off, const float *sa,
                              const float *sb, void *C, long ldc, hipStream_t stream) {
    const int nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (nblk == 0) return hipSuccess;
    dim3 grid(nblk), block(64 * WM * WN);
    const bool nt = (long)M * N * 4 <= (256L << 20);  // outputs up to 256 MiB: streaming stores
    auto go = [&](auto NT) {
        constexpr int nts = decltype(NT)::value;
        switch (out_mode) {
            case 0:
                hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, WM, WN, STAGES, OCC, 0, nts>), grid, block, 0,
                                   stream, A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K);
                break;
            case 1:
                hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, WM, WN, STAGES, OCC, 1, nts>), grid, block, 0,
                                   stream, A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K);
                break;
            default:
                hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, WM, WN, STAGES, OCC, 2, nts>), grid, block, 0,
                                   stream, A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K);
                break;
        }
    };
    if (nt) go(IC<1>{});
    else go(IC<0>{});
    return hipGetLastError();
}

// The kernel addresses each operand with 32-bit per-lane offsets: split the
// problem into row bands of A and column bands of B whose byte spans stay
// below 2^31.
template <int BM, int BN, int WM, int WN, int STAGES, int OCC>
static hipError_t launch_split(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                               const int8_t *B, long ldb, const int32_t *col_off, const float *sa,
                               const float *sb, void *C, long ldc, hipStream_t stream) {
    const long LIM = 1L << 31;
    long mband = lda > 0 ? LIM / lda : M, nband = ldb > 0 ? LIM / ldb : N;
    mband = mband >= M ? M : (mband / BM) * BM;
    nband = nband >= N ? N : (nband / BN) * BN;
    if (mband <= 0 || nband <= 0) return hipErrorInvalidValue;
    const size_t esz = 4;  // int32 or float output
    for (long m = 0; m < M; m += mband) {
        for (long n = 0; n < N; n += nband) {
            const int mm = (int)(M - m < mband ? M - m : mband);
            const int nn = (int)(N - n < nband ? N - n : nband);
            hipError_t e = launch_icfg<BM, BN, WM, WN, STAGES, OCC>(
                out_mode, mm, nn, K, A + m * lda, lda, B + n * ldb, ldb, col_off ? col_off + n : nullptr,
                sa ? sa + m : nullptr, sb ? sb + n : nullptr,
                (char *)C + (m * ldc + n) * esz, ldc, stream);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

__global__ void igemm_tiles_zero_kernel(int *ctr) {
    if (threadIdx.x < IGEMM_TILE_CTRS) ctr[threadIdx.x] = 0;
}

hipError_t launch_igemm_tiles_init(int *ctr, hipStream_t s) {
    hipLaunchKernelGGL(igemm_tiles_zero_kernel, dim3(1), dim3(64), 0, s, ctr);
    return hipGetLastError();
}

hipError_t launch_igemm(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                        const int8_t *Bpk, long ldb, const int32_t *col_off, const float *sa,
                        const float *sb, void *C, long ldc, int *tile_ctr, hipStream_t stream) {
    if (K % 256 != 0 || lda % 16 != 0 || ldb < K) return hipErrorInvalidValue;
    // Tile choice (measured on the 350M-class and gemm_bench shapes):
    //  * outputs beyond 256 MiB (the 50257-vocab head): persistent
    //    producer/consumer kernels, the stores of one tile draining under the
    //    next; 128x128 row-class tiles when rows start off 128-byte lines,
    //    256x128 tiles otherwise;
    //  * 256x256 tiles with 8 waves when they still cover most of the 256 CUs
    //    (K = 1024 projections: fewer operand bytes per output); 256x192 when
    //    those fill the CUs clearly better (4096 x 3072: 256 tiles, one round,
    //    against 192 of 256x256; +2.5-2.8% on that shape, bit-identical);
    //  * one round of 128x128 tiles (2048^3, the K = 4096 down projection,
    //    the attention output projection): igemm_kg_kernel, one tile per
    //    workgroup (same-box alternation against the persistent kernel:
    //    2048^3 12.18 against 12.60 us, FF2 19.02 against 20.75 us);
    //  * producer/consumer 128x128 tiles when those fill the chip over
    //    several rounds (row classes when rows start off 128-byte lines);
    //  * 64x64 otherwise, and for K = 0 (the epilogue alone).
    const long t256 = (long)((M + 255) / 256) * ((N + 255) / 256);
    const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    const bool huge = (long)M * N * 4 > (256L << 20);
    if (K > 0 && t256 >= 192 && huge) {
        // rows off 128-byte lines (the 50257-float head): row-class 128x128
        // tiles, whose stores are whole lines, on the persistent 16x16x64
        // kernel (head 4096 x 50257 x 1024, same box: 308-313 us against
        // 392-397 us for plain 256x128 tiles on igemm_wp_kernel and 311 us
        // for row classes there; bit-identical)
        if (classes_fill(M, ldc, C, 128))
            return launch_kgp<4, 2>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C, ldc, true, tile_ctr,
                                    stream);
        return launch_wp<256, 128, 4, 2, 3>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C,
                                            ldc, false, stream);
    }
    if (K > 0 && t256 >= 192) {
        const long t192 = (long)((M + 255) / 256) * ((N + 191) / 192);
        const double area = (double)M * N;
        const double f256 = area / ((double)((t256 + 255) / 256 * 256) * 256 * 256);
        const double f192 = area / ((double)((t192 + 255) / 256 * 256) * 256 * 192);
        if (f192 > f256 + 0.05)
            return launch_split<256, 192, 4, 2, 2, 1>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa,
                                                      sb, C, ldc, stream);
        return launch_split<256, 256, 4, 2, 2, 1>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa,
                                                  sb, C, ldc, stream);
    }
    // one round of 128x128 tiles (about one per CU): the K-grouped 16x16x64
    // kernel, two K groups once K is long (K >= 4096: a third fewer LDS
    // fragment bytes per K tile, one exchange at the end), one otherwise
    if (K > 0 && t128 >= 256 && t128 <= device_cus()) {
        if (K >= 4096)
            return launch_kg<4, 4, 2>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C, ldc, stream);
        return launch_kg<4, 2, 1>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C, ldc, stream);
    }
    if (K > 0 && t128 >= 256)
        return launch_wp<128, 128, 4, 2, 3>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C,
                                            ldc, classes_fill(M, ldc, C, 128), stream);
    return launch_split<64, 64, 2, 2, 4, 1>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C,
                                            ldc, stream);
}

// Copy A into a Kd-wide buffer (Kd >= K) padded with 0x80 (zero after re-centring; the
// packed weights are zero there as well).
__global__ void pad_a_u8_kernel(const uint8_t *__restrict__ A, long lda, int M, int K,
                                uint8_t *__restrict__ dst, int K16) {
    long total = (long)M * K16;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total;
         i += (long)gridDim.x * blockDim.x) {
        int m = (int)(i / K16), k = (int)(i % K16);
        dst[i] = k < K ? A[(long)m * lda + k] : (uint8_t)0x80;
    }
}

hipError_t launch_pad_a_u8(const uint8_t *A, long lda, int M, int K, uint8_t *dst, int K16,
                           hipStream_t stream) {
    long total = (long)M * K16;
    if (total == 0) return hipSuccess;
    int blocks = (int)((total + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(pad_a_u8_kernel, dim3(blocks), dim3(256), 0, stream, A, lda, M, K, dst, K16);
    return hipGetLastError();
}

}  // namespace pcl
