// Prefill FP8 GEMM for gfx950: y[M,N] = x[M,K] * W^T with W as E4M3FN codes
// and FP32 block scales, BF16 MFMA with FP32 accumulation (the reference's
// WMMA GEMM, src/optimized.cu:24-40, at the rounding point bf16(decode(c)*s)
// of src/optimized.cu:32), optionally with the gate/up + SwiGLU epilogue
// (src/engine.cpp:415).
//
// Workgroup: 4 waves, one per SIMD, 256 (M) x 256 (weight rows) tile (128 x
// 256 for M <= 128, see Geo).  Each wave owns all 256 rows of M and 64 weight
// rows: 8 x 2 accumulators of
// v_mfma_f32_32x32x16_bf16 held in AGPRs.  Owning the whole M extent makes the
// dequantization cost per MFMA minimal (every code is converted once per
// workgroup, 2 VALU per MFMA), and the 64-row width keeps the A-fragment LDS
// reads at one 16-byte read per two MFMAs.
//
// Data movement (K advances 64 per step, so a 128-K scale block is 2 steps):
//   A (BF16 activations): direct-to-LDS buffer loads (buffer_load_dwordx4 ...
//     lds), coalesced 8 rows x 128 B per instruction, into a 3-stage ring of
//     256 x 128 B; the 16-byte chunks of a row are XOR-swizzled (ga) so the
//     16 rows read by a quarter-wave of a fragment load hit distinct banks.
//     All 4 waves share it; one barrier per step, in the middle of the step.
//   B (FP8 codes): each wave DMAs its own 64 rows x 64 B per step (16 rows x
//     64 B per instruction) into a private 3-slot LDS ring (swizzle gb), reads
//     them back in the MFMA B-operand layout and dequantizes them in registers
//     one step ahead.  No B data crosses waves, so B needs no barrier.
//   Scales: one dword per lane per 128-K block, loaded a step ahead.
// The K index within a step is permuted identically for A and B (lane half h
// of sub-step s covers k = 32*(s/2) + 16h + 8*(s%2) + [0,8)), which changes
// only the FP32 summation order inside one MFMA.
//
// The steady state of a step is an explicit instruction sequence (one inline
// asm statement per instruction): 64 MFMAs, each followed by two dequant
// VALU instructions, with the next sub-step's LDS fragment reads, the DMAs and
// the B reads placed in fixed MFMA slots and hand-counted s_waitcnt.  The
// waits list the registers their loads filled as in/out operands, so the
// compiler neither reads nor reuses a register before its data has arrived,
// and every load into registers is retired before the loop's back edge.
#pragma once
#include <utility>

#include "device.hpp"

namespace fp8lin {
namespace gemm_fp8 {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int WN = 64, BN = 256, BK = 64;
constexpr int NT = 2;
constexpr int THREADS = 256;
constexpr int B_SLOT = WN * 64;  // 4 KiB: 64 rows x 64 codes
constexpr int B_WAVE = 3 * B_SLOT;

// The tile's M extent: MT fragments of 32 rows.  MT = 8 (256 rows) is the
// tile described above; MT = 4 (128 rows) serves launches of M <= 128 rows,
// where a 256-row tile is at least half padding: the same K loop with half
// the MFMAs per sub-step, so each code's dequantization (still once per
// workgroup) costs 4 VALU per MFMA instead of 2.
template <int MT>
struct Geo {
    static_assert(MT == 4 || MT == 8, "tile heights of 128 or 256 rows");
    static constexpr int BM = 32 * MT;
    static constexpr int A_STAGE = BM * 128;  // BM rows x 64 BF16
    static constexpr int A_BYTES = 3 * A_STAGE;
    static constexpr int LDS_BYTES = A_BYTES + 4 * B_WAVE;  // 144 KiB (MT 8) or 96 KiB (MT 4)
    static constexpr int SLOT_FLOATS = BM * BN;             // one split partial
    static constexpr int MFMAS = 2 * MT;                    // per sub-step
    static constexpr int DQ = 16 / MT;                      // dequant instructions per MFMA
    // Sub-step-0 slots of the 4 B DMAs (the 2 scale loads of odd steps sit
    // in slots MT + 1 and MT + 3, after that slot's DMA).
    static constexpr bool b_dma_at(int m) { return MT >= 8 ? (m >= MT && ((m - MT) & 1) == 0) : m >= MT; }
    static constexpr int b_dma_index(int m) { return MT >= 8 ? (m - MT) >> 1 : m - MT; }
    // Vector-memory operations issued after a step's last scale load: the
    // B DMAs in later slots of sub-step 0 and the MT A DMAs of sub-step 2.
    static constexpr int VM_AFTER_SCALE = (MT >= 8 ? 2 : 0) + MT;
    // Sub-step of the 4 code reads of B(kt+2): the last with at least 4
    // MFMAs after them before the next step's first wait (that DMA is
    // complete from sub-step 1's wait on).
    static constexpr int BRAW_SUB = MT >= 8 ? 3 : 2;
};
constexpr int kBMMax = Geo<8>::BM;

// Chunk swizzles: A rows hold 8 chunks of 16 B (slot = chunk ^ ga(row)), B
// rows 4 chunks (slot = chunk ^ gb(row)).  For any 16 consecutive rows read
// at one chunk index both keep the 16-byte slots on distinct LDS banks.
__device__ __forceinline__ int ga(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int gb(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

// Raw buffer descriptor as four SGPRs (inline-asm operand form).
__device__ __forceinline__ i32x4 make_desc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    i32x4 d;
    d.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    d.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xffff);
    d.z = __builtin_amdgcn_readfirstlane((int)bytes);
    d.w = 0x00020000;
    return d;
}

// ---- one instruction each ----
__device__ __forceinline__ void mfma(f32x16& acc, const u32x4& a, const u32x4& b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// The MFMAs are inline asm, so the compiler's hazard recognizer does not see
// that their accumulators are still being written when the epilogue reads
// them: wait for the last MFMA to finish (a 32x32x16 MFMA is 16 passes of 4
// cycles; 80 wait states leave margin), and tie every accumulator to that
// wait so no accumulator read is scheduled above it.
template <int ROWS, int COLS>
__device__ __forceinline__ void mfma_drain(f32x16 (&acc)[ROWS][COLS]) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\t"
                 "s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+a"(acc[0][0]));
#pragma unroll
    for (int i = 0; i < ROWS; ++i)
#pragma unroll
        for (int j = 0; j < COLS; ++j)
            if (i | j) asm volatile("" : "+a"(acc[i][j]));
}

// acc = 0 written straight into the accumulator registers (an MFMA of zero
// operands with a zero addend), so cleared accumulators never pass through
// VGPRs.
__device__ __forceinline__ void mfma_zero(f32x16& acc, const u32x4& zero) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=a"(acc) : "v"(zero));
}
template <int OFF>
__device__ __forceinline__ void ds_read(u32x4& d, uint32_t addr) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "i"(OFF));
}
// 64 lanes x 16 B from global (voff + soff, bounds-checked) into LDS
// [m0v, m0v + 1024), lane l at m0v + 16 l.
__device__ __forceinline__ void dma16(uint32_t m0v, uint32_t voff, i32x4 desc, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 ::"s"(m0v), "v"(voff), "s"(desc), "s"(soff) : "memory", "m0");
}
// The same with the non-temporal policy, for weight codes that one launch
// reads once (the decode and small-M streams).  Measured on MI355X: a DMA
// stream in the small-M kernels' patterns moves 10-15% more bytes per second
// from HBM with it (the 75968-row head 66 -> 57 us, 128-byte pieces; the
// gate/up codes in 512-byte row pieces 17.1 -> 15.5 us), about the rate of
// non-temporal register loads.  Data that several workgroups read (the
// activations, the prefill GEMM's tiles) keeps the default policy.
__device__ __forceinline__ void dma16_nt(uint32_t m0v, uint32_t voff, i32x4 desc, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 ::"s"(m0v), "v"(voff), "s"(desc), "s"(soff) : "memory", "m0");
}
__device__ __forceinline__ void buf_load1(float& d, uint32_t voff, i32x4 desc, int soff) {
    asm volatile("buffer_load_dword %0, %1, %2, %3 offen" : "=v"(d) : "v"(voff), "s"(desc), "s"(soff));
}
template <int N>
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory"); }
template <int N>
__device__ __forceinline__ void wait_lgkm() { asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory"); }
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// Waits that also redefine the registers their loads filled (see header).
template <int N>
__device__ __forceinline__ void wait_lgkm_a(u32x4 (&a)[8]) {
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7])
                 : "i"(N)
                 : "memory");
}
template <int N>
__device__ __forceinline__ void wait_lgkm_a(u32x4 (&a)[4]) {
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]) : "i"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_lgkm_ab(u32x4 (&a)[8], u32x4 (&b)[NT][2]) {
    asm volatile("s_waitcnt lgkmcnt(%12)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]),
                   "+v"(b[0][0]), "+v"(b[0][1]), "+v"(b[1][0]), "+v"(b[1][1])
                 : "i"(N)
                 : "memory");
}
template <int N>
__device__ __forceinline__ void wait_lgkm_ab(u32x4 (&a)[4], u32x4 (&b)[NT][2]) {
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0][0]), "+v"(b[0][1]), "+v"(b[1][0]),
                   "+v"(b[1][1])
                 : "i"(N)
                 : "memory");
}
template <int N>
__device__ __forceinline__ void wait_lgkm_braw(u32x4 (&b)[2][NT][2]) {
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(b[0][0][0]), "+v"(b[0][0][1]), "+v"(b[0][1][0]), "+v"(b[0][1][1]), "+v"(b[1][0][0]),
                   "+v"(b[1][0][1]), "+v"(b[1][1][0]), "+v"(b[1][1][1])
                 : "i"(N)
                 : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm2(float (&v)[NT]) {
    asm volatile("s_waitcnt vmcnt(%2)" : "+v"(v[0]), "+v"(v[1]) : "i"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm4(float (&v)[NT], float (&u)[NT]) {
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(v[0]), "+v"(v[1]), "+v"(u[0]), "+v"(u[1]) : "i"(N) : "memory");
}

template <int MT>
struct State {
    f32x16 acc[MT][NT];
    u32x4 af[2][MT];       // A fragments of two sub-steps
    u32x4 bf[2][NT][4];    // dequantized B fragments [step parity][frag][sub-step]
    u32x4 braw[2][NT][2];  // codes [step parity][frag][chunk pair]
    float bsc[2][NT];      // scales [128-K block parity][frag]
    f32x2 tp[2];           // dequant temporaries
    float tm[4];
};

// Instruction K (0..127) of one step's dequantization: unit K/16 = (frag j,
// sub-step ss), two code words of 4 each:
//   v_cvt_pk_f32_fp8 lo, hi  ->  4 x v_mul_f32 by the scale  ->  2 x
//   v_cvt_pk_bf16_f32 (round to nearest even): bf16(decode(c) * s).
template <int K, int RB, int BD, int MT>
__device__ __forceinline__ void dequant_op(State<MT>& st, const float (&sc)[NT]) {
    constexpr int unit = K / 16, r = K % 16;
    constexpr int j = unit / 4, ss = unit % 4;
    constexpr int wi = r / 8, q = r % 8;
    const u32x4& src = st.braw[RB][j][ss >> 1];
    const uint32_t w = (ss & 1) ? (wi ? src.w : src.z) : (wi ? src.y : src.x);
    if constexpr (q == 0) asm volatile("v_cvt_pk_f32_fp8 %0, %1" : "=v"(st.tp[0]) : "v"(w));
    if constexpr (q == 1) asm volatile("v_cvt_pk_f32_fp8_sdwa %0, %1 src0_sel:WORD_1" : "=v"(st.tp[1]) : "v"(w));
    if constexpr (q >= 2 && q <= 5) {
        constexpr int e = q - 2;
        asm volatile("v_mul_f32 %0, %1, %2" : "=v"(st.tm[e]) : "v"(st.tp[e >> 1][e & 1]), "v"(sc[j]));
    }
    if constexpr (q == 6 || q == 7) {
        constexpr int e = (q - 6) * 2;
        uint32_t o;
        asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(o) : "v"(st.tm[e]), "v"(st.tm[e + 1]));
        st.bf[BD][j][ss][wi * 2 + (q - 6)] = o;
    }
}

template <int MT>
struct Ctx {
    i32x4 dx, dw, ds;
    uint32_t aoff[MT];  // A DMA lane offsets (k = 0)
    uint32_t boff[4];   // B DMA lane offsets (k = 0)
    uint32_t soff[NT];  // scale row offsets
    uint32_t ard[4];    // A fragment read address per sub-step, stage 0
    uint32_t brd[2];    // B read address per chunk pair, slot 0
    uint32_t m0a, m0b;  // this wave's DMA LDS bases, stage / slot 0
    int scol;           // bytes per 128-K scale block in a scale row (4, or 0 for per-row scales)
};

// LDS positions of one step; the mod-3 rings are rotated at run time.
struct Ring {
    uint32_t ar, an, aw;  // A stages kt%3 (read), (kt+1)%3 (next), (kt+2)%3 (DMA)
    uint32_t bw, br;      // B slots kt%3 (DMA), (kt+2)%3 (read)
    __device__ __forceinline__ void advance() {
        const uint32_t t = ar;
        ar = an;
        an = aw;
        aw = t;
        br = bw;
        bw = bw == 2 * B_SLOT ? 0u : bw + B_SLOT;
    }
};

// Step kt, T = kt % 4.
//   A: read stage kt%3; after the mid-step barrier DMA A(kt+2) into stage
//      (kt+2)%3; in sub-step 3 read step kt+1's first fragments.
//   B: DMA B(kt+3) into slot kt%3; dequantize B(kt+1) from braw[(kt+1)&1];
//      in sub-step 3 (2 for 128-row tiles) read B(kt+2) from slot (kt+2)%3 into braw[kt&1].
//   Scales: odd steps load block (kt+3)/2 into bsc[block&1]; step kt
//      dequantizes with block (kt+1)/2.
// Per sub-step, slot m (one MFMA, then DQ dequant instructions) also carries:
//   m < MT: the next sub-step's A fragment m (LDS read);
//   sub-step 0: the 4 B DMAs (Geo::b_dma_at), and on odd steps the 2 scale
//     loads in slots MT + 1, MT + 3;
//   sub-step 2, m >= MT: A DMA m - MT;
//   sub-step BRAW_SUB, MT <= m < MT + 4: the 4 code reads of B(kt+2).
template <int MT, int T>
__device__ __forceinline__ void kstep(State<MT>& st, const Ctx<MT>& c, const Ring& rg, int kt) {
    using Gm = Geo<MT>;
    constexpr int RB_DQ = (T + 1) & 1, RB_RD = T & 1;
    constexpr int BC = T & 1, BD = BC ^ 1;
    constexpr int SB_DQ = ((T + 1) / 2) & 1;
    constexpr bool SLOAD = T & 1;
    constexpr int SB_LD = ((T + 3) / 2) & 1;
    constexpr int NS = SLOAD ? 2 : 0;
    constexpr bool PREV_SLOAD = !(T & 1);
    constexpr int SB_PREV = ((T + 2) / 2) & 1;
    const int kB = (kt + 3) * BK;
    const int kA = (kt + 2) * BK * 2;
    const int sS = ((kt + 3) >> 1) * c.scol;
    uint32_t ard[4];
#pragma unroll
    for (int q = 1; q < 4; ++q) ard[q] = c.ard[q] + rg.ar;
    ard[0] = c.ard[0] + rg.an;
    const uint32_t brd0 = c.brd[0] + rg.br, brd1 = c.brd[1] + rg.br;
    const uint32_t m0b = c.m0b + rg.bw, m0a = c.m0a + rg.aw;

    [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
        ([&]() __attribute__((always_inline)) {
            constexpr int s = S;
            if constexpr (s == 0)
                wait_lgkm_ab<0>(st.af[0], st.braw[RB_DQ]);
            else
                wait_lgkm_a<0>(st.af[s & 1]);
            [&]<int... M>(std::integer_sequence<int, M...>) __attribute__((always_inline)) {
                ([&]() __attribute__((always_inline)) {
                    constexpr int m = M;
                    constexpr int i = m >> 1, j = m & 1;
                    mfma(st.acc[i][j], st.af[s & 1][i], st.bf[BC][j][s]);
                    [&]<int... D>(std::integer_sequence<int, D...>) __attribute__((always_inline)) {
                        (dequant_op<(s * Gm::MFMAS + m) * Gm::DQ + D, RB_DQ, BD>(st, st.bsc[SB_DQ]), ...);
                    }(std::make_integer_sequence<int, Gm::DQ>{});
                    if constexpr (m < MT) {
                        if constexpr (s < 3)
                            ds_read<m * 4096>(st.af[(s + 1) & 1][m], ard[s + 1]);
                        else
                            ds_read<m * 4096>(st.af[0][m], ard[0]);
                    }
                    if constexpr (s == 0 && Gm::b_dma_at(m)) {
                        constexpr int g = Gm::b_dma_index(m);
                        dma16(m0b + g * 1024, c.boff[g], c.dw, kB);
                    }
                    if constexpr (SLOAD && s == 0 && (m == MT + 1 || m == MT + 3))
                        buf_load1(st.bsc[SB_LD][(m - MT - 1) >> 1], c.soff[(m - MT - 1) >> 1], c.ds, sS);
                    if constexpr (s == 2 && m >= MT)
                        dma16(m0a + (m - MT) * 1024, c.aoff[m - MT], c.dx, kA);
                    if constexpr (s == Gm::BRAW_SUB && m >= MT && m < MT + 4) {
                        constexpr int jj = (m - MT) >> 1, cp = (m - MT) & 1;
                        ds_read<jj * 2048>(st.braw[RB_RD][jj][cp], cp ? brd1 : brd0);
                    }
                }(), ...);
            }(std::make_integer_sequence<int, Gm::MFMAS>{});
            if constexpr (s == 1) {
                // A(kt+1), the previous step's last DMA, has landed (issued
                // after it: this step's 4 B DMA and NS scale loads).
                if constexpr (PREV_SLOAD)
                    wait_vm2<4 + NS>(st.bsc[SB_PREV]);
                else
                    wait_vm<4 + NS>();
                barrier();
            }
        }(), ...);
    }(std::make_integer_sequence<int, 4>{});
}

// Work decomposition.  The output is cut into BM x 256 tiles (L = 0..T-1,
// walked GROUP_M tile rows at a time so that tiles running together on one
// XCD share A and B slices in its L2).  The grid is persistent: G workgroups
// (one per CU, G a multiple of 8) loop over work units u = bid, bid + G, ...
//  - units [0, fpad) are whole tiles, written to y.  Unit u runs on XCD
//    u % 8 (the dispatcher deals workgroups round-robin over the XCDs), and
//    takes tile L = (u % 8) * (fpad / 8) + u / 8, so each XCD owns a
//    contiguous tile range (fpad = full rounded up to a multiple of 8; units
//    whose L >= full do nothing);
//  - units [fpad, fpad + rtiles * splits) cover the tail tiles full..T-1, each
//    cut into `splits` K ranges (whole 256-K chunks, spread evenly).  Their
//    FP32 sums go to partial slot r * splits + s (BM x 256 floats each, in
//    the tile's own row/column order) and tail_reduce_kernel adds the splits
//    in order, rounds once and applies the epilogue.
// The host picks the tile height BM (plan.bm) and full = T, rtiles = 0 when
// splitting would not pay (see gemm.hip), so most launches write every tile
// directly.
constexpr int kXcds = 8;
constexpr int kGroupM = 8;
constexpr int kMaxSplits = 8;

struct Plan {
    int bm;              // tile height: 256 or 128 rows of M
    int mtiles, ntiles;  // tile grid (ntiles counts 256-row weight blocks, or 128 output pairs for SwiGLU)
    int full;            // whole tiles
    int fpad;            // full rounded up to a multiple of 8
    int rtiles, splits;  // tail tiles and their K ranges
    int units;           // fpad + rtiles * splits
};

__device__ __forceinline__ void tile_coords(int L, int mtiles, int ntiles, int& mt, int& nt) {
    const int per_group = kGroupM * ntiles;
    const int g = L / per_group;
    const int first_m = g * kGroupM;
    const int gsize = min(kGroupM, mtiles - first_m);
    const int r = L - g * per_group;
    mt = first_m + r % gsize;
    nt = r / gsize;
}

// K range of split s of `splits`: whole 256-K chunks, spread evenly.
__device__ __forceinline__ void split_range(int K, int s, int splits, int& kbeg, int& klen) {
    const int chunks = K / 256;
    const int c0 = (int)((int64_t)s * chunks / splits), c1 = (int)((int64_t)(s + 1) * chunks / splits);
    kbeg = 256 * c0;
    klen = 256 * (c1 - c0);
}

struct Unit {
    int mtile, ntile, kbeg, klen;
    int slot;  // partial slot, or -1 for a whole tile
};

__device__ __forceinline__ bool unit_of(int u, const Plan& p, int K, Unit& w) {
    if (u < p.fpad) {
        const int L = (u % kXcds) * (p.fpad / kXcds) + u / kXcds;
        if (L >= p.full) return false;
        tile_coords(L, p.mtiles, p.ntiles, w.mtile, w.ntile);
        w.kbeg = 0;
        w.klen = K;
        w.slot = -1;
        return true;
    }
    const int v = u - p.fpad;
    const int r = v / p.splits, s = v % p.splits;
    tile_coords(p.full + r, p.mtiles, p.ntiles, w.mtile, w.ntile);
    split_range(K, s, p.splits, w.kbeg, w.klen);
    w.slot = v;
    return true;
}

// Weight row of local column rr (0..63) of wave `wave` in tile column
// block nt, or -1 past the end.  SwiGLU tiles hold 128 gate rows and the
// 128 matching up rows: wave w's columns 0..31 are gate rows, 32..63 up.
template <bool SWIGLU>
__device__ __forceinline__ int64_t weight_row(int nt, int wave, int rr, int N) {
    if constexpr (SWIGLU) {
        const int D = N >> 1;
        const int o = nt * (BN / 2) + wave * (WN / 2) + (rr & 31);
        return o < D ? (rr < 32 ? (int64_t)o : (int64_t)D + o) : -1;
    } else {
        const int64_t n = (int64_t)nt * BN + wave * WN + rr;
        return n < N ? n : -1;
    }
}

// Buffer descriptors and lane offsets of one unit (its tile and K range).
template <bool SWIGLU, int MT>
__device__ __forceinline__ void setup(Ctx<MT>& c, const Unit& w, const uint16_t* x, const uint8_t* wt, const float* scales,
                                      int S, int M, int N, int K, int wave, int lane, uint32_t lds0) {
    const int h = lane >> 5, l32 = lane & 31;
    constexpr int BM = Geo<MT>::BM, A_BYTES = Geo<MT>::A_BYTES;
    const int m0 = w.mtile * BM;
    const int sbeg = S == 1 ? 0 : w.kbeg / 128;
    // The buffers start at kbeg (rows keep the stride K), so the step offsets
    // of the loop are relative to it.
    c.dx = make_desc(x + w.kbeg, (uint32_t)((int64_t)M * K * 2 - (int64_t)w.kbeg * 2));
    c.dw = make_desc(wt + w.kbeg, (uint32_t)((int64_t)N * K - w.kbeg));
    c.ds = make_desc(scales + sbeg, (uint32_t)((int64_t)N * S * 4 - (int64_t)sbeg * 4));
    c.scol = S == 1 ? 0 : 4;
    // A DMA instruction ii of wave w fills rows 8G..8G+7 (G = MT w + ii) of a
    // stage: lane -> row 8G + lane/8, LDS slot lane%8 <- chunk slot ^ ga(row).
#pragma unroll
    for (int ii = 0; ii < MT; ++ii) {
        const int r = 8 * (MT * wave + ii) + (lane >> 3);
        const int ch = (lane & 7) ^ ga(r);
        const int m = m0 + r;
        c.aoff[ii] = m < M ? (uint32_t)((int64_t)m * K * 2 + ch * 16) : kBufferOob;
    }
    c.m0a = __builtin_amdgcn_readfirstlane(lds0 + wave * MT * 1024);
    // B DMA instruction gi fills rows 16gi..16gi+15 of a slot: lane -> row
    // 16gi + lane/4, LDS slot lane%4 <- chunk slot ^ gb(row).
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
        const int rr = 16 * gi + (lane >> 2);
        const int ch = (lane & 3) ^ gb(rr);
        const int64_t n = weight_row<SWIGLU>(w.ntile, wave, rr, N);
        c.boff[gi] = n >= 0 ? (uint32_t)(n * K + ch * 16) : kBufferOob;
    }
    c.m0b = __builtin_amdgcn_readfirstlane(lds0 + A_BYTES + wave * B_WAVE);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int64_t n = weight_row<SWIGLU>(w.ntile, wave, 32 * j + l32, N);
        c.soff[j] = n >= 0 ? (uint32_t)(n * S * 4) : kBufferOob;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int ch = 4 * (s >> 1) + 2 * h + (s & 1);
        c.ard[s] = lds0 + l32 * 128 + 16 * (ch ^ ga(l32));
    }
#pragma unroll
    for (int cp = 0; cp < 2; ++cp)
        c.brd[cp] = lds0 + A_BYTES + wave * B_WAVE + l32 * 64 + 16 * ((2 * cp + h) ^ gb(l32));
}

// Prologue loads of a unit, in the order the first step needs them: A(0)
// into stage 0, B(0) and B(1) into slots 0 and 1, scale blocks 0 and 1, then
// A(1) into stage 1 and B(2) into slot 2 (the last MT + 4 loads).
template <int MT>
__device__ __forceinline__ void issue_prologue(State<MT>& st, const Ctx<MT>& c) {
#pragma unroll
    for (int ii = 0; ii < MT; ++ii) dma16(c.m0a + ii * 1024, c.aoff[ii], c.dx, 0);
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) dma16(c.m0b + p * B_SLOT + gi * 1024, c.boff[gi], c.dw, p * BK);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        buf_load1(st.bsc[0][j], c.soff[j], c.ds, 0);
        buf_load1(st.bsc[1][j], c.soff[j], c.ds, c.scol);
    }
#pragma unroll
    for (int ii = 0; ii < MT; ++ii) dma16(c.m0a + Geo<MT>::A_STAGE + ii * 1024, c.aoff[ii], c.dx, BK * 2);
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) dma16(c.m0b + 2 * B_SLOT + gi * 1024, c.boff[gi], c.dw, 2 * BK);
}

// The rest of the prologue once A(0), B(0), B(1) and the scales have landed
// (at most the MT + 4 loads of A(1) and B(2), or later stores, still in
// flight): B(0) dequantized, B(1) codes and step 0's first A fragments read;
// the accumulators cleared.  Step 0 first touches A(1) and B(2) after its
// mid-step wait, which leaves only that step's own loads in flight, so
// those two need no wait here; the kernel starts its first step about 1 us
// earlier than with everything waited for (M = 512: 4.3 against 5.5 us
// from launch to the first MFMA).
template <int MT>
__device__ __forceinline__ void finish_prologue(State<MT>& st, const Ctx<MT>& c) {
    wait_vm4<MT + 4>(st.bsc[0], st.bsc[1]);
    barrier();
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int cp = 0; cp < 2; ++cp) {
            ds_read<0>(st.braw[0][j][cp], c.brd[cp] + j * 2048);
            ds_read<B_SLOT>(st.braw[1][j][cp], c.brd[cp] + j * 2048);
        }
    wait_lgkm_braw<0>(st.braw);
    [&]<int... K2>(std::integer_sequence<int, K2...>) __attribute__((always_inline)) {
        (dequant_op<K2, 0, 0>(st, st.bsc[0]), ...);
    }(std::make_integer_sequence<int, 128>{});
#pragma unroll
    for (int i = 0; i < MT; ++i) ds_read<0>(st.af[0][i], c.ard[0] + i * 4096);
    const u32x4 zero{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) mfma_zero(st.acc[i][j], zero);
    wait_lgkm_a<0>(st.af[0]);
}

// Requirements (checked by the launcher): K % 256 == 0; x and w 16-byte
// aligned; S == K/128 or S == 1; M*K*2, N*K, N*S*4 and (M + 256)*ldy*2
// below 2^31; plan.bm == 32 * MT.  When SWIGLU, N is the number of weight rows
// (gate rows [0, N/2), up rows [N/2, N)) and y is [M, N/2].  part: rtiles *
// splits partial slots of BM x 256 floats (unused when rtiles == 0).
template <int MT, bool SWIGLU>
__global__ __launch_bounds__(256, 1) void gemm_fp8_kernel(const uint16_t* __restrict__ x,
                                                          const uint8_t* __restrict__ w,
                                                          const float* __restrict__ scales, int S,
                                                          uint16_t* __restrict__ y, int ldy, int M, int N,
                                                          int K, Plan plan, float* __restrict__ part) {
    extern __shared__ __align__(16) uint16_t smem[];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

    int u = blockIdx.x;
    Unit cur;
    while (u < plan.units && !unit_of(u, plan, K, cur)) u += gridDim.x;
    if (u >= plan.units) return;
    using Gm = Geo<MT>;
    Ctx<MT> c;
    State<MT> st;
    setup<SWIGLU>(c, cur, x, w, scales, S, M, N, K, wave, lane, lds0);
    issue_prologue(st, c);
    finish_prologue(st, c);

    for (;;) {
        // ---- K loop, 4 steps per iteration; only LDS DMA stays in flight
        // across the back edge.
        const int KT = cur.klen / BK;
        Ring rg{0u, (uint32_t)Gm::A_STAGE, (uint32_t)(2 * Gm::A_STAGE), 0u, (uint32_t)(2 * B_SLOT)};
        for (int kt = 0; kt < KT; kt += 4) {
            kstep<MT, 0>(st, c, rg, kt);
            rg.advance();
            kstep<MT, 1>(st, c, rg, kt + 1);
            rg.advance();
            kstep<MT, 2>(st, c, rg, kt + 2);
            rg.advance();
            kstep<MT, 3>(st, c, rg, kt + 3);
            rg.advance();
            // step kt+3 read step kt+4's fragments and B(kt+5) (LDS) and loaded
            // scale block (kt+6)/2 into bsc[1], followed by VM_AFTER_SCALE DMA
            // (10 for 256-row tiles, 4 for 128).
            wait_lgkm_ab<0>(st.af[0], st.braw[1]);
            wait_vm2<Gm::VM_AFTER_SCALE>(st.bsc[1]);
        }
        // The last steps prefetched past the K range (the next K, or zeros
        // past the buffers); their LDS DMA must land before the rings are
        // reused or the workgroup's LDS is freed.
        wait_vm<0>();
        mfma_drain(st.acc);

        // ---- next unit: once every wave is done reading the rings, its
        // prologue loads run under this unit's epilogue.
        int un = u + gridDim.x;
        Unit nxt;
        while (un < plan.units && !unit_of(un, plan, K, nxt)) un += gridDim.x;
        const bool more = un < plan.units;
        const int ep_mtile = cur.mtile, ep_ntile = cur.ntile, ep_slot = cur.slot;
        if (more) {
            barrier();
            setup<SWIGLU>(c, nxt, x, w, scales, S, M, N, K, wave, lane, lds0);
            issue_prologue(st, c);
        }

        // ---- epilogue: acc[i][j][r] = C[32i + 8(r/4) + 4h + r%4][wave col 32j + l32].
        // Each accumulator pair is copied to VGPRs by an empty asm before its
        // elements are read: with the accumulators live around the unit loop,
        // element reads straight from them made the register allocator move
        // every accumulator through scratch memory.
        if (ep_slot >= 0) {
            // FP32 partial of a split tail tile: rows and columns in tile order.
            const rsrc_t rp = make_rsrc(part + (int64_t)ep_slot * Gm::SLOT_FLOATS, (uint32_t)(Gm::SLOT_FLOATS * 4));
            uint32_t voff[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j) voff[j] = (uint32_t)((4 * h * BN + wave * WN + 32 * j + l32) * 4);
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                f32x16 av[NT] = {st.acc[i][0], st.acc[i][1]};
                asm volatile("" : "+v"(av[0]), "+v"(av[1]));
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int dr = 32 * i + 8 * (r >> 2) + (r & 3);
#pragma unroll
                    for (int j = 0; j < NT; ++j) {
                        // copy the element first: __builtin_bit_cast of a vector
                        // element reads element 0 with hipcc (ROCm 7.2)
                        const float a = av[j][r];
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, a), rp, (int)voff[j],
                                                              dr * BN * 4, 0);
                    }
                }
            }
        } else {
            // Stores go through a buffer bounded to the M x ldy output: rows
            // >= M fall outside it and columns past the end get an
            // out-of-range lane offset.
            const int row0 = ep_mtile * Gm::BM + 4 * h;
            const rsrc_t ry = make_rsrc(y, (uint32_t)((int64_t)M * ldy * 2));
            if constexpr (SWIGLU) {
                const int D = N >> 1;
                const int col = ep_ntile * (BN / 2) + wave * (WN / 2) + l32;
                const uint32_t voff = col < D ? (uint32_t)(((int64_t)row0 * ldy + col) * 2) : kBufferOob;
                // 16 outputs per batch: with one wave per SIMD nothing else
                // hides an output's dependency chain (exp2, rcp, the window
                // test, two BF16 roundings), so independent outputs are
                // computed side by side.
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    uint32_t gu[16];
                    uint16_t v[16];
                    f32x16 a0 = st.acc[i][0], a1 = st.acc[i][1];
                    asm volatile("" : "+v"(a0), "+v"(a1));
#pragma unroll
                    for (int r = 0; r < 16; ++r) gu[r] = pack_bf16x2(f32x2{a0[r], a1[r]});
                    swiglu_bf16_batch<16>(gu, v);
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int dr = 32 * i + 8 * (r >> 2) + (r & 3);
                        __builtin_amdgcn_raw_buffer_store_b16(v[r], ry, (int)voff, dr * ldy * 2, 0);
                    }
                }
            } else {
                // both accumulator columns of a row at once, in the order the
                // SwiGLU epilogue reads them (fewer accumulators live at a time)
                uint32_t voff[NT];
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    const int col = ep_ntile * BN + wave * WN + 32 * j + l32;
                    voff[j] = col < N ? (uint32_t)(((int64_t)row0 * ldy + col) * 2) : kBufferOob;
                }
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    f32x16 a0 = st.acc[i][0], a1 = st.acc[i][1];
                    asm volatile("" : "+v"(a0), "+v"(a1));
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int dr = 32 * i + 8 * (r >> 2) + (r & 3);
                        const uint32_t p = pack_bf16x2(f32x2{a0[r], a1[r]});
                        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(p & 0xffffu), ry, (int)voff[0],
                                                              dr * ldy * 2, 0);
                        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(p >> 16), ry, (int)voff[1], dr * ldy * 2,
                                                              0);
                    }
                }
            }
        }
        if (!more) break;
        u = un;
        cur = nxt;
        finish_prologue(st, c);
    }
}

// Tail reduction: tail tile r of the plan gets out = bf16(sum over s in
// order of its partial slots) at the unsplit epilogue's rounding points, or
// with SWIGLU y = swiglu(bf16(gate sum), bf16(up sum)), for rows < M and
// columns inside the output.  Four tile columns per thread.
template <int MT, bool SWIGLU>
__global__ __launch_bounds__(256) void tail_reduce_kernel(const float* __restrict__ part, Plan plan, int M, int N,
                                                          uint16_t* __restrict__ y, int64_t ldy) {
    constexpr int BM = Geo<MT>::BM, SLOT = Geo<MT>::SLOT_FLOATS;
    constexpr int CG = SWIGLU ? 32 : 64;  // 4-column groups per tile row
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)plan.rtiles * BM * CG) return;
    const int r = (int)(idx / (BM * CG));
    const int rem = (int)(idx % (BM * CG));
    const int row = rem / CG, cg = rem % CG;
    int mt, nt;
    tile_coords(plan.full + r, plan.mtiles, plan.ntiles, mt, nt);
    const int m = mt * BM + row;
    if (m >= M) return;
    // tile-local column of the first of the four (the gate column for SWIGLU)
    const int lc = SWIGLU ? (cg / 8) * WN + 4 * (cg % 8) : 4 * cg;
    const float* p = part + (int64_t)r * plan.splits * SLOT + row * BN + lc;
    auto sum = [&](int off) __attribute__((always_inline)) -> f32x4 {
        f32x4 s = *reinterpret_cast<const f32x4*>(p + off);
        for (int k = 1; k < plan.splits; ++k) s += *reinterpret_cast<const f32x4*>(p + (int64_t)k * SLOT + off);
        return s;
    };
    const f32x4 a = sum(0);
    uint16_t* dst = y + (int64_t)m * ldy;
    uint16_t o[4];
    int col, lim;
    if constexpr (SWIGLU) {
        const f32x4 g = sum(32);
        lim = N >> 1;
        col = nt * (BN / 2) + (cg / 8) * (WN / 2) + 4 * (cg % 8);
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = swiglu_bf16_bits(f32_to_bf16_bits(a[q]), f32_to_bf16_bits(g[q]));
    } else {
        lim = N;
        col = nt * BN + lc;
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = f32_to_bf16_bits(a[q]);
    }
    // the four outputs in one 8-byte store where they are all inside the
    // output and aligned (about 0.5 us of the M = 512 QKV-gate call's 11 us
    // reduce against four 2-byte stores)
    if (col + 3 < lim && (reinterpret_cast<uintptr_t>(dst + col) & 7) == 0) {
        uint2 v;
        v.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
        v.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
        *reinterpret_cast<uint2*>(dst + col) = v;
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (col + q < lim) dst[col + q] = o[q];
    }
}

// True when the kernel's requirements hold (see gemm_fp8_kernel).
inline bool supported(const uint16_t* x, const void* w, int S, int64_t ldy, int64_t M, int64_t N, int64_t K) {
    const int64_t lim = (int64_t)1 << 31;
    return K % 256 == 0 && K > 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(w) % 16 == 0 && (S == 1 || S == K / 128) && M * K * 2 < lim &&
           N * K < lim && N * (int64_t)S * 4 < lim && (M + kBMMax) * ldy * 2 < lim;
}

}  // namespace gemm_fp8
}  // namespace fp8lin
