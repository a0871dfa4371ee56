// Decode chain: the one-row (M = 1) linear layers of a decode step in one
// launch.
//
// The reference runs a decode step as one captured graph
// (src/engine.cpp:522-539) of Engine::step's per-projection linear calls
// (src/engine.cpp:401-421), each an fp8_linear GEMV.  On MI355X each such
// GEMV launch pays a ramp at its start (the first HBM data arrives about
// 2 us after the first loads) and a drain at its end (the last waves finish
// alone), and the next launch cannot start its loads before the previous one
// has drained.  Here the links share one grid:
//
//  - the grid holds every link's workgroups in link order; a workgroup is
//    4 waves, each owning two items of the decode GEMV's ring form
//    (gemv_kernel.hpp): an item is 2 weight rows (a gate/up pair with
//    SwiGLU) of up to 5 K steps of 1024 codes, or 1 row of up to 9 steps;
//  - workgroups are dispatched in grid order on each XCD, so the first
//    workgroups of link L + 1 start while link L drains: they issue their
//    first item's code loads -- which never depend on the activations --
//    then wait for the link whose output they read, then load the
//    activations and the second item's codes, so HBM has the second items'
//    bytes to stream while the first items are summed.  Waiting workgroups hold
//    slots that link L no longer needs (all of its workgroups on that XCD
//    were dispatched before them), so the waits always end;
//  - a link that reads an earlier link's output waits for that link: each
//    workgroup adds 1 to one of its link's 256 slot counters (workgroup w of
//    the link to slot w mod 256, each slot in its own 128-byte line: adds to
//    one address serialize at about 50 ns each, so one counter for the
//    head's 9496 workgroups took 0.5 ms) once its 4 waves' outputs have been
//    stored (coherent sc1 stores, completed: s_waitcnt);
//  - the first wave of a dependent workgroup reads its XCD's word of the
//    link (in its own 256-byte line): if it records this call, the link is
//    complete.  Otherwise the link's first 8 workgroups (one per XCD, as
//    workgroups are dealt to the XCDs round robin) poll the sum of the 256
//    slots (coherent loads, 4 per lane) until every workgroup of that link
//    has added its 1 and then record the call in their XCD's word; the
//    others poll that word, and the slots themselves every 64th time (so a
//    wait ends whatever the dealing).  The other waves wait at a barrier.
//    Then every workgroup reads its activations into LDS with coherent
//    (sc1) direct-to-LDS loads, which read what other XCDs stored without
//    invalidating this XCD's L2 (an invalidate per XCD and dependency cost
//    about 5 us);
//  - the counters are 64-bit and never reset: each call adds to slot s the
//    number n_s of the link's workgroups that map to it.  A workgroup of a
//    link that waits reads its own slot when it starts -- below (t + 1) n_s,
//    as it has not added its 1 yet -- which gives the call's index t, and
//    waits for the slots of the link it reads to sum to (t + 1) G (G: that
//    link's workgroups).  Only a link that a later link waits for stores its
//    outputs coherently and waits for their completion before its add (a
//    workgroup that waits for its stores holds its slot longer: every
//    workgroup doing so made a single 75968-row link 18% slower); a link
//    that only waits adds without waiting (its counter only gives t).  A
//    workspace thus counts one chain shape: word 1 records it (FNV-1a of
//    the links' workgroup counts and waits), and a chain of another shape
//    skips its waits and counts them in word 0 instead of waiting for
//    counts that never come;
//  - waits are bounded: a poll loop that runs kSpinLimit times adds 1 to a
//    timeout count and goes on (its outputs are then wrong; the host reads
//    the count), so the grid always drains.
//
// Measured (graph replay, weights rotated over 600 MB): links with no waits
// stream at 6.7 TB/s in one launch (QKV-gate + gate/up + down + head,
// 86 us against 93 us as four GEMV launches), but each wait costs about
// 8 us: the producer's last adds reach the pollers 2-3 us after its last
// stores, its last workgroups start late (when earlier ones free their
// slots) and finish last, and the waiting workgroups' activations land only
// after the code loads queued before them.  The same four links each after
// the previous take 108 us (124 us with one item per wave, when the
// workgroups that held the compute units at the wake left HBM idle until
// they finished; 110 us with polls 512 clocks apart instead of 256); a
// graph of four GEMV launches remains the faster strict chain.
//
// Numerics: each row is summed exactly as the decode GEMV's one-row ring
// kernel sums it (lane l takes the 16-code chunks l + 64 j in step order,
// v_cvt_pk_f32_fp8, x scale, v_cvt_pk_bf16_f32, v_dot2_f32_bf16, then a
// butterfly across the wave), so each link's output equals fp8lin_linear's
// (fp8lin_linear_swiglu's) at M = 1 bit for bit.
#include <algorithm>

#include "gemm_fp8.hpp"
#include "gemv_kernel.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

constexpr int kWPG = 4;          // waves per workgroup
constexpr int kItems = 2;        // items per wave: item it of wave w of workgroup b is g = (b kItems + it) kWPG + w
constexpr int kMaxSteps = 9;     // K <= 9216
constexpr int kXDmas = kMaxSteps * 2;   // 1 KiB direct-to-LDS loads of a link's activations
constexpr int kXBytes = kXDmas * 1024;  // a workgroup's activations in LDS
constexpr int kXcds = 8;
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t kSlotPollEvery = 64;

using gemm_fp8::i32x4;
using gemm_fp8::make_desc;

struct LinkDev {
    const uint8_t* codes;
    const float* scales;
    const uint16_t* x;
    uint16_t* y;
    int N, K, S;
    int mode;    // 0: 2 rows (a gate/up pair with SwiGLU) x <= 5 steps; 1: 1 row x <= 9 steps
    int swiglu;
    int after;   // link whose outputs this link's x holds (waited for), or -1
    int groups;  // items of the link
    int wg0;     // first workgroup of the link
    int wgs;     // workgroups of the link
    int publish; // a later link waits for this one
};

// Sync words (64-bit): word 0 counts timed-out or skipped waits; word 1 the
// chain's shape (signature); slot s of link L at
// cnt_word(L, s); XCD x's word of link L at xcd_word(nlinks, L, x).
constexpr int kCountSlots = 256;
constexpr int kLineWords = 16;  // 128 bytes
__host__ __device__ constexpr size_t cnt_word(int L, int s) { return kLineWords + ((size_t)L * kCountSlots + s) * kLineWords; }
__host__ __device__ constexpr size_t xcd_word(int nlinks, int L, int x) {
    return cnt_word(nlinks, 0) + ((size_t)L * kXcds + x) * 2 * kLineWords;
}

struct ChainArgs {
    LinkDev link[kChainMaxLinks];
    int nlinks;
    uint64_t* sync;
    uint64_t sig;  // the chain's shape (links' workgroups and waits), never 0
};

__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

// 64 lanes x 16 B from global into LDS [m0v, m0v + 1024) through L2; with
// COHERENT, agent-scope loads (sc1), which read what other XCDs stored
// without an L2 invalidate.
template <bool COHERENT>
__device__ __forceinline__ void dma16(uint32_t m0v, uint32_t voff, i32x4 desc) {
    if constexpr (COHERENT)
        asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen sc1 lds" ::"s"(m0v), "v"(voff),
                     "s"(desc)
                     : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0v), "v"(voff), "s"(desc)
                     : "memory", "m0");
}

// One output: a coherent (sc1) store when another link reads it.
__device__ __forceinline__ void store_out(uint16_t* p, uint16_t v, int coherent) {
    if (coherent)
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}

__device__ __forceinline__ uint64_t load_sync(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return (int)(v & (kXcds - 1));
}

// One wave's kItems items of link k (item it: g + kWPG it), each R rows
// (slot_row of the ring kernel) x up to NS steps.  A link that waits: the
// first item's chunks, then `wait` (the dependency, all 4 waves together),
// then `x_dma` (the activations into LDS `xs`), then the other items'
// chunks, and the activations and first item landed before the sums start;
// otherwise, as the ring kernel orders them, `x_dma` first, every item's
// chunks, and the wait only for the activations.  Then sums each item's rows
// in the ring kernel's order with the activations from LDS (step s at
// xs + 2048 s: lane l's 16 BF16 of chunk l + 64 s at +16 l and +1024 + 16 l)
// and stores them.
template <int R, int NS, bool SWIGLU, class Wait, class XDma>
__device__ __forceinline__ void run_item(const LinkDev& k, int64_t g, int lane, const uint8_t* xs, Wait&& wait,
                                         XDma&& x_dma) {
    using gemv::Chunk;
    const gemv::Buffers b = gemv::make_buffers(k.x, k.codes, k.scales, k.S, 1, k.N, k.K, true);
    int64_t rows[kItems][R];
    bool ok[kItems][R];
#pragma unroll
    for (int it = 0; it < kItems; ++it)
#pragma unroll
        for (int r = 0; r < R; ++r) rows[it][r] = gemv::slot_row<R, SWIGLU>(g + kWPG * it, r, k.N, ok[it][r]);
    const int chunks = k.K >> 4;
    const int steps = (chunks + kWave - 1) / kWave;
    const bool dep = k.after >= 0;
    Chunk<true> ring[kItems][NS][R];
    auto load_item = [&](int it) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const int c = lane + j * kWave;
#pragma unroll
            for (int r = 0; r < R; ++r)
                gemv::load_chunk_buf<true, 2>(ring[it][j][r], b, k.S, rows[it][r], k.K, c << 4,
                                              ok[it][r] && c < chunks);
        }
    };
    if (dep) {
        // the first item's codes, the wait, the activations, the other items'
        // codes; then the activations and everything older
        load_item(0);
        wait();
        x_dma();
#pragma unroll
        for (int it = 1; it < kItems; ++it) load_item(it);
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"(2 * R * NS * (kItems - 1)) : "memory");
    } else {
        // the activation DMAs are older than the 2 R NS chunk loads per item
        x_dma();
#pragma unroll
        for (int it = 0; it < kItems; ++it) load_item(it);
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"(2 * R * NS * kItems) : "memory");
    }
    wg_barrier();
#pragma unroll
    for (int it = 0; it < kItems; ++it) {
        float acc[R][1];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][0] = 0.0f;
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            // each step's LDS reads stay in its step
#pragma unroll
            for (int r = 0; r < R; ++r) asm volatile("" : "+v"(acc[r][0])::"memory");
            const u32x4 lo = *reinterpret_cast<const u32x4*>(xs + 2048 * j + 16 * lane);
            const u32x4 hi = *reinterpret_cast<const u32x4*>(xs + 2048 * j + 1024 + 16 * lane);
            const uint32_t xv[1][8] = {{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w}};
            float nxt[R][1];
#pragma unroll
            for (int r = 0; r < R; ++r) nxt[r][0] = acc[r][0];
            gemv::accumulate<R, 1, true>(nxt, ring[it][j], xv);
            const bool live = j < steps;
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][0] = live ? nxt[r][0] : acc[r][0];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][0] = wave_sum(acc[r][0]);
        if (lane == 0) {
            if constexpr (SWIGLU) {
                if (ok[it][0])
                    store_out(k.y + rows[it][0],
                              swiglu_bf16_bits(f32_to_bf16_bits(acc[0][0]), f32_to_bf16_bits(acc[1][0])), k.publish);
            } else {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (ok[it][r]) store_out(k.y + rows[it][r], f32_to_bf16_bits(acc[r][0]), k.publish);
            }
        }
    }
}

__global__ __launch_bounds__(64 * kWPG) void chain_kernel(ChainArgs a) {
    __shared__ __align__(16) uint8_t xs[kXBytes];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int b = blockIdx.x;
    int L = 0;
    while (L + 1 < a.nlinks && b >= a.link[L + 1].wg0) ++L;
    const LinkDev& k = a.link[L];
    const int64_t g = (int64_t)(b - k.wg0) * kWPG * kItems + wave;
    uint64_t* sync = a.sync;
    const int w = b - k.wg0, slot = w % kCountSlots;
    // the call index, from this workgroup's own slot (see header)
    const uint64_t t = wave == 0 && k.after >= 0
                           ? load_sync(sync + cnt_word(L, slot)) /
                                 (uint64_t)(k.wgs / kCountSlots + (slot < k.wgs % kCountSlots ? 1 : 0))
                           : 0;
    // word 1 holds the shape of the chain the counters count (0: none yet);
    // a workspace used before for another chain fails fast instead of
    // waiting for counts that never come
    uint64_t cfg = 0;
    if (wave == 0 && (k.after >= 0 || b == 0)) cfg = load_sync(sync + 1);
    if (b == 0 && wave == 0 && lane == 0 && cfg == 0)
        __hip_atomic_store(sync + 1, a.sig, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    auto wait = [&]() __attribute__((always_inline)) {
        {
            if (wave == 0) {
                uint64_t* xw = sync + xcd_word(a.nlinks, L, xcc_id());
                if (cfg != 0 && cfg != a.sig) {
                    if (lane == 0)
                        __hip_atomic_fetch_add(sync, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else if (load_sync(xw) < t + 1) {
                    const LinkDev& d = a.link[k.after];
                    const uint64_t target = (t + 1) * (uint64_t)d.wgs;
                    uint32_t n = 0;
                    for (;;) {
                        // the link's first kXcds workgroups (one per XCD as
                        // workgroups are dealt out round robin) poll the
                        // slots; the others the XCD word, and the slots
                        // only every kSlotPollEvery-th time
                        if (w >= kXcds && (n % kSlotPollEvery) != kSlotPollEvery - 1) {
                            if (load_sync(xw) >= t + 1) break;
                            if (++n == kSpinLimit) {
                                if (lane == 0)
                                    __hip_atomic_fetch_add(sync, (uint64_t)1, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
                                break;
                            }
                            __builtin_amdgcn_s_sleep(4);
                            continue;
                        }
                        uint64_t part = 0;
#pragma unroll
                        for (int i = 0; i < kCountSlots / kWave; ++i)
                            part += load_sync(sync + cnt_word(k.after, lane + kWave * i));
                        uint32_t lo = (uint32_t)part, hi = (uint32_t)(part >> 32);
                        uint64_t sum = part;
#pragma unroll
                        for (int dd = 32; dd >= 1; dd >>= 1) {
                            const uint64_t o = (uint64_t)(uint32_t)__shfl_xor((int)lo, dd, kWave) |
                                               ((uint64_t)(uint32_t)__shfl_xor((int)hi, dd, kWave) << 32);
                            sum += o;
                            lo = (uint32_t)sum;
                            hi = (uint32_t)(sum >> 32);
                        }
                        if (sum >= target) break;
                        if (++n == kSpinLimit) {
                            if (lane == 0)
                                __hip_atomic_fetch_add(sync, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(4);
                    }
                    // record it for the call (the activations are then
                    // read with coherent loads: no L2 invalidate)
                    if (lane == 0) __hip_atomic_store(xw, t + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            wg_barrier();
        }
    };
    // the link's activations into LDS: 2 KiB per step of 1024, DMA q by wave
    // q mod 4
    auto x_dma = [&]() __attribute__((always_inline)) {
        const i32x4 rx = make_desc(k.x, (uint32_t)((int64_t)k.K * 2));
        const int chunks = k.K >> 4;
        const int dmas = 2 * ((chunks + kWave - 1) / kWave);
        const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)xs);
        for (int q = wave; q < dmas; q += kWPG) {
            const int s = q >> 1, h = q & 1;
            const int ch = lane + 64 * s;
            const uint32_t off = ch < chunks ? (uint32_t)(ch * 32 + 16 * h) : kBufferOob;
            if (k.after >= 0)
                dma16<true>(base + 1024 * q, off, rx);
            else
                dma16<false>(base + 1024 * q, off, rx);
        }
    };

    if (k.mode == 0) {
        if (k.swiglu)
            run_item<2, 5, true>(k, g, lane, xs, wait, x_dma);
        else
            run_item<2, 5, false>(k, g, lane, xs, wait, x_dma);
    } else {
        run_item<1, kMaxSteps, false>(k, g, lane, xs, wait, x_dma);
    }
    if (k.publish) {
        // this workgroup's outputs have completed, then its add
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        wg_barrier();
    }
    if ((k.publish || k.after >= 0) && wave == 0 && lane == 0)
        __hip_atomic_fetch_add(sync + cnt_word(L, slot), (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

bool chain_link_supported(int64_t N, int64_t K, int64_t S, bool swiglu) {
    const int64_t lim = (int64_t)1 << 31;
    return N > 0 && K > 0 && K % 16 == 0 && K <= 1024 * kMaxSteps && (!swiglu || (N % 2 == 0 && K <= 5120)) &&
           (S == 1 || S == (K + 127) / 128) && N * K < lim && N * S * 4 < lim;
}

size_t chain_sync_words(int nlinks) { return xcd_word(nlinks, nlinks, 0); }

hipError_t launch_chain(const ChainLink* links, int nlinks, uint64_t* sync, hipStream_t stream) {
    ChainArgs a{};
    a.nlinks = nlinks;
    a.sync = sync;
    int wg = 0;
    for (int L = 0; L < nlinks; ++L) {
        const ChainLink& s = links[L];
        LinkDev& d = a.link[L];
        d.codes = s.codes;
        d.scales = s.scales;
        d.x = s.x;
        d.y = s.y;
        d.N = (int)s.N;
        d.K = (int)s.K;
        d.S = (int)s.S;
        d.swiglu = s.swiglu ? 1 : 0;
        d.after = s.after;
        d.mode = (s.swiglu || s.K <= 5120) ? 0 : 1;
        d.groups = (int)(d.mode == 0 ? (s.swiglu ? s.N / 2 : (s.N + 1) / 2) : s.N);
        d.wg0 = wg;
        d.wgs = (d.groups + kWPG * kItems - 1) / (kWPG * kItems);
        d.publish = 0;
        if (s.after >= 0) a.link[s.after].publish = 1;
        wg += d.wgs;
    }
    uint64_t sig = 1469598103934665603ull;  // FNV-1a over the counted shape
    auto mix = [&](int64_t v) {
        for (int i = 0; i < 8; ++i) sig = (sig ^ (uint64_t)((v >> (8 * i)) & 0xff)) * 1099511628211ull;
    };
    mix(nlinks);
    for (int L = 0; L < nlinks; ++L) {
        mix(a.link[L].wgs);
        mix(a.link[L].after);
    }
    a.sig = sig | 1;
    hipLaunchKernelGGL(chain_kernel, dim3(wg), dim3(64 * kWPG), 0, stream, a);
    return hipGetLastError();
}

}  // namespace fp8lin
