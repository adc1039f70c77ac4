// gfx950 (MI355X) split-KV paged decode and its log-sum-exp merge.
//
//   decode_split_kernel_*  per-segment attention over HND pages (decode_kernels.cuh:123-403)
//   decode_merge_kernel    LSE-weighted merge of split rows      (decode_kernels.cuh:409-432)
//
// Split kernel design (one wave64 = one work unit of the persistent plan):
//   * A wave streams its own contiguous list of (row, kv head, token range)
//     segments in steps of NG = 16 or 32 tokens (two 16-token halves), DEPTH
//     steps of K/V in flight (in registers, or in the LDS stage below). The
//     pages of a step are looked up another DEPTH steps ahead, so an HBM load
//     never waits on the block table.
//   * K is held token-major: in each 16-token half, lane (c, kb) holds token
//     c and a quarter of its dims. That is the A-operand layout of
//     v_mfma_f32_16x16x32_f16 for S^T = K Q^T with the G query heads sharing
//     the kv head as B columns.
//   * V is held dim-major: lane (c, kb) holds tokens 4kb..4kb+3 of each half,
//     dims 8c..8c+7. After a v_perm regroup that is the B operand of the P V
//     MFMA (MFMA j <-> dims 8c + j): 16x16x16 for 16-token steps, 16x16x32
//     with the two halves as one k-block for 32-token steps. The S^T
//     accumulators are already the A-operand layout of P, so P never leaves
//     registers.
//   * fp16 loads K and V straight into those layouts. FP8 rows are 128 B, so
//     the same layouts would split every row over many lanes' small pieces;
//     the FP8 kernel instead loads each 16-token half fully coalesced (16 B
//     per lane, 8 whole rows per instruction) straight into a per-wave LDS
//     stage (LDS-destination buffer loads, one step in flight) and reads the
//     layouts from there into registers at the top of each step, after which
//     the next step's loads are issued into the stage, so they arrive during
//     the step's arithmetic. The stage's 16-byte chunks are XOR-swizzled by row
//     (the swizzle is applied to the source addresses, since lane i's bytes
//     land at 16 i), so the column-wise K reads are free of bank conflicts.
//   * When the page size is a power of two >= 16, a 16-token half lies in one
//     page: one wave-uniform table read (a scalar load) per half, and each
//     load is a raw buffer load from an SGPR resource based at the half's
//     first row, with constant lane offsets. The resource's range is the
//     half's valid tokens, so loads past a segment's end (and every load of a
//     slot past the unit's last step) return zeros without touching memory,
//     and every slot issues the same loads, which keeps the hardware wait
//     counts exact. Smaller
//     pages go through the LDS stage for both element types: pages of whole
//     1 KiB parts (fp16 P = 4 and 8, FP8 P = 8) with one resource per part,
//     any other size with each lane loading a row whose page it looks up
//     itself (the step's table entries spread over the lanes, handed out by
//     ds_bpermute).
//   * Online softmax in base 2 with a lazy running max: probabilities use a
//     reference max per head that only moves (with the exact O/l rescale) when
//     a score exceeds it by more than 2^8, so the cross-lane max reduction is
//     paid at a segment's first step and then almost never. P <= 256 stays far
//     inside fp16 range and l in fp32.
//   * FP8 E4M3 is widened to fp16 in registers (exact); k_scale folds into the
//     softmax scale and v_scale into the output normalization.
//   * Q of each segment is fetched compactly (G x 256 B across the wave) with
//     the segment's first K/V loads and expanded to the B-operand layout
//     through a per-wave LDS slot once per segment; on the LDS-stage paths it
//     lands there with the same LDS-destination loads, ahead of the K / V.
//   * Split rows are merged by the split kernel itself when the plan allows
//     (block_merge 1 and 2): a unit's split segments are only its first and
//     last, so each wave keeps at most two partials (and their LSEs) in LDS;
//     after one barrier every thread of the block merges one head-dim element
//     of each split row. A row inside the block (e.g. 32 rows x 8 kv heads x
//     8192 tokens over 2048 units) is then complete; a row that spans blocks
//     (up to 8) leaves one device-coherent partial per block, and the last
//     of its blocks to arrive (a per-row counter) combines them, in block
//     order. No merge launch is needed. Otherwise (rows over more blocks, or
//     caller plans that do not keep a row's segments in consecutive units)
//     every split segment's partial goes to the plan's workspace for the
//     merge kernel.

#include "pa_device.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <type_traits>

// Compile-time tuning knobs, per cache element type.
// Tokens per step (16 or 32), the same on every page path.
#ifndef PA_FP16_STEP
#define PA_FP16_STEP 16
#endif
#ifndef PA_FP8_STEP
#define PA_FP8_STEP 32
#endif
// Steps of K/V in flight per wave.
#ifndef PA_FP16_DEPTH
#define PA_FP16_DEPTH 1
#endif
#ifndef PA_FP8_DEPTH
#define PA_FP8_DEPTH 2
#endif
// 1: K/V loads are non-temporal (streamed once, kept out of the caches).
#ifndef PA_FP16_NONTEMPORAL
#define PA_FP16_NONTEMPORAL 1
#endif
#ifndef PA_FP8_NONTEMPORAL
#define PA_FP8_NONTEMPORAL 1
#endif
// Waves per SIMD the split kernel is register-budgeted for.
#ifndef PA_FP16_WAVES_PER_EU
#define PA_FP16_WAVES_PER_EU 2
#endif
#ifndef PA_FP8_WAVES_PER_EU
#define PA_FP8_WAVES_PER_EU 2
#endif
// K lane layout. 1: lane (c, kb) load j holds token c, dims 32j + 8kb .. +7
// (MFMA j's A operand in natural dim order; one load instruction covers 16
// rows x 64 B (fp16) / 32 B (fp8) contiguous). 0: lane (c, kb) holds dims
// 32kb .. 32kb+31 in 16-byte loads (half the fp8 load instructions; each
// instruction touches 4 x 16 B spread over every row).
#ifndef PA_FP16_K_NATURAL
#define PA_FP16_K_NATURAL 1
#endif
#ifndef PA_FP8_K_NATURAL
#define PA_FP8_K_NATURAL 0
#endif
// FP8, page sizes that are powers of two >= 16: 1 = K and V are fetched with
// fully coalesced 16-byte loads (each instruction 8 whole 128-byte rows) and
// put into the MFMA lane layouts through an 8 KiB LDS stage per wave.
#ifndef PA_FP8_LDS_STAGE
#define PA_FP8_LDS_STAGE 1
#endif
// The same for fp16 pages of 16 tokens and more (4 rows per 1 KiB load).
#ifndef PA_FP16_LDS_STAGE
#define PA_FP16_LDS_STAGE 0
#endif
// 1: the LDS stage stores 16-byte chunk j of row r at chunk position
// j ^ (r % chunks per row), so that the column-wise reads of the MFMA lane
// layouts hit distinct banks; 0: chunks in natural order (the comparison build
// behind the bank-conflict counters).
#ifndef PA_STAGE_SWIZZLE
#define PA_STAGE_SWIZZLE 1
#endif
// 1: every LDS-staged path fills the stage with LDS-destination loads
// (buffer / global_load_dwordx4 ... lds: 16 bytes per lane land at M0 + 16 *
// lane, no VGPRs, no ds_write), one step in flight; 0: loads into VGPRs, then
// ds_write, with the path's tuned depth.
#ifndef PA_LDS_DMA
#define PA_LDS_DMA 1
#endif

// Diagnostic builds only (PA_STAMPS=1): per-block s_memrealtime stamps of the
// split kernel's phases, read back with pa_debug_stamps.
#ifndef PA_STAMPS
#define PA_STAMPS 0
#endif
#if PA_STAMPS
__device__ unsigned long long pa_stamps[4096 * 24];
extern "C" int pa_debug_stamps(void* host, unsigned long bytes) {
    return static_cast<int>(hipMemcpyFromSymbol(host, HIP_SYMBOL(pa_stamps), bytes, 0, hipMemcpyDeviceToHost));
}
#endif
__device__ __forceinline__ void stamp(int k) {
#if PA_STAMPS
    if ((threadIdx.x & 63) == 0 && blockIdx.x < 4096) pa_stamps[blockIdx.x * 24 + k] = __builtin_amdgcn_s_memrealtime();
#else
    (void)k;
#endif
}
// The shader clock counter (s_memtime), for the CU's effective clock between
// two stamps of the same wave.
__device__ __forceinline__ void stamp_clock(int k) {
#if PA_STAMPS
    if ((threadIdx.x & 63) == 0 && blockIdx.x < 4096) pa_stamps[blockIdx.x * 24 + k] = __builtin_amdgcn_s_memtime();
#else
    (void)k;
#endif
}

namespace pa {
namespace {

constexpr int   kWaves        = kBlockUnits;   // waves (work units) per block
constexpr float kRescaleSlack = 8.0f;   // log2 headroom of the lazy running max
constexpr float kLog2e        = 1.4426950408889634f;
// The cache-policy operand of buffer loads (2 = non-temporal).
template <bool NT> constexpr int kAux = NT ? 2 : 0;
// ... and of a device-coherent load (sc1: served from the device's coherence
// point, like a relaxed agent-scope atomic load).
constexpr int kAuxCoherent = 16;

template <int EB> struct Tune {
    static constexpr int  step  = EB == 2 ? PA_FP16_STEP : PA_FP8_STEP;
    static constexpr int  depth = EB == 2 ? PA_FP16_DEPTH : PA_FP8_DEPTH;
    static constexpr bool nt    = EB == 2 ? PA_FP16_NONTEMPORAL != 0 : PA_FP8_NONTEMPORAL != 0;
    static constexpr bool knat  = EB == 2 ? PA_FP16_K_NATURAL != 0 : PA_FP8_K_NATURAL != 0;
    static constexpr bool stage = EB == 2 ? PA_FP16_LDS_STAGE != 0 : !knat && PA_FP8_LDS_STAGE != 0;
};
static_assert(Tune<2>::step == 16 || Tune<2>::step == 32, "fp16 step must be 16 or 32");
static_assert(Tune<1>::step == 16 || Tune<1>::step == 32, "fp8 step must be 16 or 32");
constexpr bool kLdsDma = PA_LDS_DMA != 0;
constexpr bool kStageSwizzle = PA_STAGE_SWIZZLE != 0;

// LDS-destination load of 16 bytes per lane: lane i's bytes land at dst + 16 i
// (AUX: the cache-policy operand, 2 = non-temporal).
template <int AUX>
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t rs, u32x4* dst, int voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)dst, 16, voffset, 0, 0,
                                             AUX);
}
template <int AUX>
__device__ __forceinline__ void lds_load16(const void* src, u32x4* dst) {
    __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)const_cast<void*>(src),
                                     (__attribute__((address_space(3))) void*)dst, 16, 0, AUX);
}
// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0] and [15:14], expcnt [6:4],
// lgkmcnt [11:8]): wait for every vector memory operation (LDS-destination
// loads included), or for every LDS / scalar memory operation.
constexpr int kWaitVm0   = 0x0F70;
constexpr int kWaitLgkm0 = 0xC07F;

// How a step finds its pages.
enum PagePath : int {
    kPagePow2 = 0,   // page_size a power of two >= 16: a 16-token half is in one page
    kPageQuad = 1,   // FP8 without the LDS stage, page_size 4 or 8: one lookup per lane
                     // for K and one for V
    kPageAny  = 2,   // FP8 without the LDS stage, any other page size: one lookup per
                     // token, integer division
    kPageRuns = 3,   // page_size 4 or 8 (fp16) / 8 (FP8 with the LDS stage): K/V through
                     // the LDS stage, one wave-uniform page per coalesced 1 KiB part
    kPageLane = 4,   // every other page size (1, 2, FP8 4, any non-power of two): K/V
                     // through the LDS stage, each lane finding the page of the row it
                     // loads (coalesced 16-byte loads at per-lane addresses)
};

// One position of a wave's schedule: the current step of the current segment.
// Every field is wave-uniform.
struct Cursor {
    int seg;
    int b, h;    // batch row, kv head
    int tok;     // first token of the step
    int t0, w;   // segment start and end (exclusive)
};

__device__ __forceinline__ void cursor_load(Cursor& c, const int4* segs) {
    const int4 s = segs[c.seg];
    c.b   = s.x;
    c.h   = s.y;
    c.tok = s.z;
    c.t0  = s.z;
    c.w   = s.w;
}

// Moves to the next step: 0 = same segment, 1 = next segment, -1 = none (the
// cursor stays on its last step).
template <int NG>
__device__ __forceinline__ int cursor_step(Cursor& c, const int4* segs, int seg_end) {
    if (__builtin_expect(c.tok + NG < c.w, 1)) {
        c.tok += NG;
        return 0;
    }
    if (c.seg + 1 >= seg_end) return -1;
    c.seg++;
    cursor_load(c, segs);
    return 1;
}

// p[i] for a wave-uniform p and i, as a scalar load: the block table is not
// written while a decode kernel runs, so it may be read through the constant
// address space, whose loads the compiler always makes scalar (the table reads
// then stay out of the vector memory counters that the LDS stage waits on).
__device__ __forceinline__ int load_uniform(const int32_t* p, int i) {
    using const_ptr = const __attribute__((address_space(4))) int32_t*;
    return ((const_ptr)(reinterpret_cast<uintptr_t>(p)))[__builtin_amdgcn_readfirstlane(i)];
}

// Block-table row of batch row b (decode_kernels.cuh:150-153).
__device__ __forceinline__ const int* table_row(const pa_decode_params& p, const int32_t* __restrict__ tbl,
                                                const int32_t* __restrict__ sid, int b) {
    const int slot = sid ? sid[b] : b;
    return tbl + static_cast<size_t>(slot) * p.block_table_stride;
}

// arr[4 * kb + i] for the heads a lane's O rows hold (kb only matters for G = 8).
template <int G>
__device__ __forceinline__ float head_pick(const float (&arr)[G], int kb, int i) {
    if constexpr (G > 4) return kb ? arr[4 + i] : arr[i];
    else return arr[i < G ? i : 0];
}

// One normalized O row (head row i of the lane's accumulators) of a split
// segment into a partial row: lane c holds dims 8c .. 8c+7.
__device__ __forceinline__ void store_row(float* row, const f32x4 (&oacc)[8], int i, float inv, int c) {
    f32x4 lo, hi;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        lo[j] = oacc[j][i] * inv;
        hi[j] = oacc[4 + j][i] * inv;
    }
    *reinterpret_cast<f32x4*>(row + 8 * c)     = lo;
    *reinterpret_cast<f32x4*>(row + 8 * c + 4) = hi;
}

// x from the lane that DPP control CTRL selects within each row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    const int v = __builtin_bit_cast(int, x);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false));
}

// Device-coherent store of the partials that blocks exchange inside one launch:
// a relaxed agent-scope atomic store, written through to the device's
// coherence point (the XCDs' L2 caches are not coherent with each other), and
// complete there once the wave's vector memory counter has drained. The
// reads use the same scope's cache policy (kAuxCoherent).
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-level merge after the split loop. slot_item holds, per wave, the
// (row, kv head) item of its first (slot 0) and last (slot 1) segment when that
// segment is a split one, else -1 (slot_seg: that segment's index); part / lse
// hold the slot's normalized partial rows and base-2 LSEs, written to LDS by
// the wave that computed them. Each thread owns one head-dim element (two for
// G = 8) of every item and reads that element of all 16 slots at once, with
// the LSEs and slot items (one LDS round trip). An item's weights
// 2^(lse - max) depend only on the slot and the head, and a wave's 64
// elements share one head, so lane j of each wave computes slot j's weight
// once (0 outside the item) and the element sums take them as wave-uniform
// operands: the base-2 LSE-weighted average of the item's partials in this
// block (decode_kernels.cuh:409-432), summed in slot order. No branch depends
// on a slot.
//
// An item whose segments all lie in this block (block_merge 1: every split
// item) is written as fp16. With block_merge 2 an item may also span blocks
// (its k-th segment runs in unit u0 + k, so it continues from the previous
// block at the block's first slot and into the next at its last): the block's
// average becomes one partial row of the item, at the workspace slot of the
// item's first segment in the block, with LSE max + log2(sum of weights).
// After every thread's stores are complete, one lane per such item adds one to
// the item's counter; the block that brings it to the item's block count
// resets it to zero and combines the item's block partials, in block order, as
// the merge kernel does (so the result does not depend on which block is
// last). Blocks never wait for each other.
template <int G>
__device__ __forceinline__ void block_merge(const pa_decode_params& p, const int32_t* __restrict__ isb,
                                            const int (*slot_item)[2], const int (*slot_seg)[2],
                                            const float (*part)[G * kHeadDim], const float (*lse)[G],
                                            int* last_lds, int tid, int lblock) {
    constexpr int NS = 2 * kWaves;
    constexpr int NO = G * kHeadDim;
    constexpr int NE = (NO + 64 * kWaves - 1) / (64 * kWaves);   // elements per thread
    static_assert(NS == 16, "the slot lanes form one DPP row");
    static_assert(kHeadDim % 64 == 0, "a wave's elements share one head");
    const int  lane  = tid & 63;
    const bool slot  = lane < NS;   // lane j holds slot j
    const bool chain = p.block_merge == 2;
    if (tid == 0) stamp(16);
    float lv[NE], pv[NE][NS];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
        const int o = tid + 64 * kWaves * e;
        if (o < NO) {
            lv[e] = lse[lane & (NS - 1)][o / kHeadDim];
#pragma unroll
            for (int j = 0; j < NS; ++j) pv[e][j] = part[j][o];
        }
    }
    const int      mine   = slot_item[(lane & (NS - 1)) >> 1][lane & 1];
    const int      myseg  = slot_seg[(lane & (NS - 1)) >> 1][lane & 1];
#if PA_STAMPS
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    if (tid == 0) stamp(17);
#endif
    const uint64_t filled = __builtin_amdgcn_ballot_w64(slot && mine >= 0);
    // Items of this block that span blocks (at most two), block-uniform.
    int ns = 0, sx0 = 0, su0 = 0, sn0 = 0, sx1 = 0, su1 = 0, sn1 = 0;
    uint64_t run = 0;
    for (uint64_t rem = filled; rem != 0; rem &= ~run) {
        const int j0 = __builtin_ctzll(rem);
        const int x  = __builtin_amdgcn_readlane(mine, j0);   // the next item
        run = __builtin_amdgcn_ballot_w64(slot && mine == x);
        const int  n     = isb[x + 1] - isb[x];
        const bool spans = chain && __builtin_popcountll(run) != n;
#if PA_STAMPS
        if (tid == 0 && rem == filled) stamp(18 + spans);
#endif
        const int  bseg  = __builtin_amdgcn_readlane(myseg, j0);   // the item's first segment here
        if (spans) {
            const int u0 = lblock * kWaves + (j0 >> 1) - (bseg - isb[x]);   // unit of its first segment
            if (ns == 0) { sx0 = x; su0 = u0; sn0 = n; }
            else { sx1 = x; su1 = u0; sn1 = n; }
            ++ns;
        }
        const bool in = (run >> lane) & 1;
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            const int o = tid + 64 * kWaves * e;
            if (o >= NO) break;
            // The item's maximum LSE over the 16 slot lanes (one DPP row):
            // swaps of neighbours and pairs in each quad, then rotations by 4
            // and 8.
            float mx = in ? lv[e] : -INFINITY;
            mx = fmaxf(mx, dpp_f32<0xB1>(mx));    // quad_perm [1,0,3,2]
            mx = fmaxf(mx, dpp_f32<0x4E>(mx));    // quad_perm [2,3,0,1]
            mx = fmaxf(mx, dpp_f32<0x124>(mx));   // row_ror:4
            mx = fmaxf(mx, dpp_f32<0x128>(mx));   // row_ror:8
            const float w = in ? exp2_fast(lv[e] - mx) : 0.f;
            float a = 0.f, den = 0.f;
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), j));
                a   = fmaf(wj, ((run >> j) & 1) ? pv[e][j] : 0.f, a);   // empty slots hold no partial
                den = den + wj;
            }
            if (!spans) {
                const int b = x / p.num_kv_heads, h = x - b * p.num_kv_heads;
                p.out[(static_cast<size_t>(b) * p.num_q_heads + h * G) * kHeadDim + o] =
                    __builtin_bit_cast(uint16_t, static_cast<_Float16>(a * (1.0f / den)));
            } else {
                store_coherent(p.partial_out + static_cast<size_t>(bseg) * NO + o, a * (1.0f / den));
                if (o % kHeadDim == 0)
                    store_coherent(p.partial_lse + static_cast<size_t>(bseg) * G + o / kHeadDim, mx + __log2f(den));
            }
        }
    }
    if (ns == 0) return;
    if (tid == 0) stamp(9);

    // Arrivals: this block's partial rows are complete at the coherence point
    // before its counters move.
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (tid == 0) stamp(10);
    if (tid < ns) {
        const int x  = tid == 0 ? sx0 : sx1;
        const int u0 = tid == 0 ? su0 : su1;
        const int n  = tid == 0 ? sn0 : sn1;
        const int nb = (u0 + n - 1) / kWaves - u0 / kWaves + 1;   // blocks the item spans
        int* ctr = p.merge_counters + x;
        const int before = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = before == nb - 1;
        if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // for the next decode
        last_lds[tid] = last;
    }
    __syncthreads();
    if (tid == 0) stamp(11);
    // The last block combines the item's block partials (block j's sits at the
    // item's first segment in block j). Thread (v, g), g = tid % NGR, takes
    // 16 bytes (4 dims) v of every NGR-th block from g on, up to 8 blocks at a
    // time, each with one coherent 16-byte load of the row and one of its LSE,
    // all issued before the first is used (one round trip), and keeps a
    // running maximum over them in block order; the NGR states of one dim
    // vector sit in adjacent lanes of one DPP row and are combined in a fixed
    // tree (lanes 1, 2 apart, then quad and half-row mirrors), so the result
    // does not depend on timing.
    constexpr int NV  = NO / 4;                  // 16-byte vectors of one block partial
    constexpr int NGR = 64 * kWaves / NV;        // lanes sharing one vector (16, 8, 4, 2 for G = 1, 2, 4, 8)
    static_assert(NGR >= 1 && NGR <= 16 && (NGR & (NGR - 1)) == 0, "the groups of a vector form one DPP row");
    const int gi = tid % NGR;
    const int vi = tid / NGR;
    const int hh = 4 * vi / kHeadDim;            // query head of the vector
    for (int i = 0; i < ns; ++i) {
        if (!last_lds[i]) continue;
        const int x  = i == 0 ? sx0 : sx1;
        const int u0 = i == 0 ? su0 : su1;
        const int n  = i == 0 ? sn0 : sn1;
        const int s0 = isb[x];
        const int j0 = u0 / kWaves, j1 = (u0 + n - 1) / kWaves;
        const int nb = j1 - j0 + 1;
        const int b = x / p.num_kv_heads, h = x - b * p.num_kv_heads;
        // The item's partial rows and LSEs, from its first segment on (byte
        // offsets fit 32 bits: n segments of NO floats).
        const __amdgpu_buffer_rsrc_t rs =
            buffer_rsrc(p.partial_out + static_cast<size_t>(s0) * NO, n * NO * static_cast<int>(sizeof(float)));
        const __amdgpu_buffer_rsrc_t rl =
            buffer_rsrc(p.partial_lse + static_cast<size_t>(s0) * G, n * G * static_cast<int>(sizeof(float)));
        float  m = -INFINITY, den = 0.f;
        f32x4  acc = {0.f, 0.f, 0.f, 0.f};
        const int per = (nb + NGR - 1) / NGR;   // blocks per group (the first groups may take one more)
        for (int k0 = 0; k0 < per; k0 += 8) {
            u32x4 raw[8];
            float ls[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int j = j0 + gi + NGR * (k0 + t);
                if (j <= j1) {
                    const int k = max(0, kWaves * j - u0);   // the block's first segment, from s0
                    raw[t] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                   rs, (k * NO + 4 * vi) * static_cast<int>(sizeof(float)), 0, kAuxCoherent));
                    ls[t] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(
                                   rl, (k * G + hh) * static_cast<int>(sizeof(float)), 0, kAuxCoherent));
                }
            }
#if PA_STAMPS
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            if (tid == 0 && i == 0 && k0 == 0) stamp(12);
#endif
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int j = j0 + gi + NGR * (k0 + t);
                if (j > j1) break;
                const float mn  = fmaxf(m, ls[t]);
                const float f   = exp2_fast(m - mn);   // 0 while m = -inf
                const float wgt = exp2_fast(ls[t] - mn);
                const f32x4 v   = __builtin_bit_cast(f32x4, raw[t]);
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[c] = fmaf(wgt, v[c], acc[c] * f);
                den = fmaf(den, f, wgt);
                m   = mn;
            }
        }
        // Combine the NGR states of the vector (a group with no block has
        // m = -inf and weighs 0).
        auto combine = [&](float m2, float d2, const f32x4& a2) {
            const float mt = fmaxf(m, m2);
            const float f1 = m == -INFINITY ? 0.f : exp2_fast(m - mt);
            const float f2 = m2 == -INFINITY ? 0.f : exp2_fast(m2 - mt);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = acc[c] * f1 + a2[c] * f2;
            den = den * f1 + d2 * f2;
            m   = mt;
        };
        auto partner_round = [&](auto ctrl) {
            constexpr int C = decltype(ctrl)::value;
            f32x4 a2;
#pragma unroll
            for (int c = 0; c < 4; ++c) a2[c] = dpp_f32<C>(acc[c]);
            combine(dpp_f32<C>(m), dpp_f32<C>(den), a2);
        };
        if (tid == 0 && i == 0) stamp(13);
        if constexpr (NGR >= 2) partner_round(std::integral_constant<int, 0xB1>{});    // quad_perm [1,0,3,2]
        if constexpr (NGR >= 4) partner_round(std::integral_constant<int, 0x4E>{});    // quad_perm [2,3,0,1]
        if constexpr (NGR >= 8) partner_round(std::integral_constant<int, 0x141>{});   // row_half_mirror
        if constexpr (NGR >= 16) partner_round(std::integral_constant<int, 0x140>{});  // row_mirror
        if (tid == 0 && i == 0) stamp(14);
        if (gi == 0) {
            const float inv = 1.0f / den;
            const f16x2 lo = {static_cast<_Float16>(acc[0] * inv), static_cast<_Float16>(acc[1] * inv)};
            const f16x2 hi = {static_cast<_Float16>(acc[2] * inv), static_cast<_Float16>(acc[3] * inv)};
            *reinterpret_cast<u32x2*>(p.out + (static_cast<size_t>(b) * p.num_q_heads + h * G) * kHeadDim + 4 * vi) =
                u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        }
        if (tid == 0 && i == 0) stamp(15);
    }
}

// ---------------------------------------------------------------------------
// Split kernel body.
//   EB    cache element bytes (2 fp16, 1 fp8)
//   G     query heads per kv head (1, 2, 4, 8)
//   NG    tokens per step (16 or 32)
//   DEPTH steps of K/V in flight per wave
//   PATH  page resolution (PagePath)
template <int EB, int G, int NG, int DEPTH, int PATH>
__device__ __forceinline__ void decode_split_body(const pa_decode_params& p, const int32_t* __restrict__ cta,
                                                  int num_units, int page_shift,
                                                  const int32_t* __restrict__ tbl, const int32_t* __restrict__ sid,
                                                  const int32_t* __restrict__ segp, const int32_t* __restrict__ isb) {
    constexpr int  NH    = NG / 16;                 // 16-token halves per step
    constexpr int  ROW   = kRowBytes<EB>;           // bytes per token row
    constexpr bool NT    = Tune<EB>::nt;
    constexpr bool KNAT  = Tune<EB>::knat;
    constexpr int  KL    = KNAT ? 8 * EB : 16;      // bytes per K load
    constexpr int  NK    = KNAT ? 4 : ROW / 64;     // K loads per lane per half
    constexpr int  KSTEP = KNAT ? 32 * EB : 16;     // byte distance between a lane's K loads
    constexpr int  KLANE = KNAT ? KL : ROW / 4;     // byte offset of k-block kb in a row
    constexpr int  VCH   = 8 * EB;                  // V bytes per lane per token (8 dims)
    constexpr int  NQ    = G > 4 ? 2 : 1;           // compact Q registers per lane
    constexpr int  NVL   = PATH == kPageAny ? 4 : 1;   // V page lookups per lane (per-lane paths)
    constexpr int  HW    = G < 4 ? G : 4;           // live O rows per writing lane
    constexpr bool STG   = PATH == kPageRuns || PATH == kPageLane ||
                           (Tune<EB>::stage && PATH == kPagePow2);   // K/V via LDS
    constexpr int  RPP   = 1024 / ROW;              // rows per coalesced 1 KiB part (4 fp16, 8 FP8)
    constexpr int  NPART = 16 / RPP;                // parts per 16-token half
    constexpr int  CPR   = ROW / 16;                // 16-byte chunks per row
    constexpr int  HCH   = 16 * CPR;                // 16-byte chunks per half (256 B per row x 16)
    constexpr bool DMA   = STG && kLdsDma;          // the stage is filled by LDS-destination loads
    // The stage's chunk permutation of row r (XOR with r % CPR).
    auto swz = [](int r) { return kStageSwizzle ? r % CPR : 0; };
    static_assert(!DMA || DEPTH == 1, "the LDS-destination stage holds one step");
    using VRaw = std::conditional_t<EB == 2, u32x4, u32x2>;
    using KRaw = std::conditional_t<KL == 16, u32x4, u32x2>;

    // Compact Q per wave (G heads x 256 B; on the LDS-destination paths filled
    // by issue() with the K / V, 1 KiB per load).
    __shared__ __attribute__((aligned(16))) u32x4 q_lds[kWaves][64 * NQ];
    __shared__ int slot_item[kWaves][2];                                     // split segments per wave
    __shared__ int slot_seg[kWaves][2];                                      // their segment indices
    __shared__ int last_lds[2];                                              // block merges a spanning item
    // LDS stage of one step per wave (STG): [K, V][half][16 rows][row bytes],
    // each row's 16-byte chunks XOR-swizzled by (row % chunks per row).
    __shared__ __attribute__((aligned(16))) u32x4 stage_lds[STG ? kWaves : 1][STG ? 2 * NH * HCH : 1];
    // Partials of split segments for the block-level merge, slot 2 * wave + sl.
    __shared__ __attribute__((aligned(16))) float part_lds[2 * kWaves][G * kHeadDim];
    __shared__ float lse_lds[2 * kWaves][G];

    if (threadIdx.x == 0) {
        stamp(0);
        stamp_clock(20);
    }
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lblock = static_cast<int>(blockIdx.x);   // units 8 lblock .. 8 lblock + 7
    const int unit   = lblock * kWaves + wave;
    const bool merge_here = p.block_merge != 0;   // block-level merge of split rows
    if (lane == 0) {
        slot_item[wave][0] = -1;
        slot_item[wave][1] = -1;
    }
    int seg_begin = 0, seg_end = 0;
    if (unit < num_units) {
        seg_begin = cta[unit];
        seg_end   = cta[unit + 1];
    }
    if (seg_begin < seg_end) {

    const int c  = lane & 15;   // MFMA column / row index within a 16-block
    const int kb = lane >> 4;   // MFMA k-block
    const int4* __restrict__ segs = reinterpret_cast<const int4*>(segp);
    const unsigned char* kbase = static_cast<const unsigned char*>(p.k_cache);
    const unsigned char* vbase = static_cast<const unsigned char*>(p.v_cache);
    const int P   = p.page_size;
    const int hkv = p.num_kv_heads;
    const int hq  = p.num_q_heads;
    const float qk_scale = p.sm_scale * p.k_scale * kLog2e;   // softmax in base 2
    const uint32_t page_bytes = static_cast<uint32_t>(hkv * P * ROW);   // one page of one pool
    // Constant lane offsets inside a 16-token half (power-of-two path).
    const int k_lane_off = c * ROW + kb * KLANE;
    const int v_lane_off = 4 * kb * ROW + c * VCH;
    // LDS-destination stage: lane i of 1 KiB part `part` lands in slot 64 part +
    // i, i.e. row RPP part + i / CPR, chunk position i % CPR, which holds
    // chunk (i % CPR) ^ (row % CPR) of that row (the swizzle moves to the
    // source): dma_chunk[part] is that chunk's byte offset within its row.
    int dma_chunk[NPART];
#pragma unroll
    for (int part = 0; part < NPART; ++part)
        dma_chunk[part] = 16 * ((lane % CPR) ^ swz(RPP * part + lane / CPR));
    u32x4* const stage = stage_lds[STG ? wave : 0];

    // ---- pipeline registers, indexed by ring slot = step index mod DEPTH
    KRaw  kr[DEPTH][NH][NK];   // K: token 16hh + c of each half
    VRaw  vr[DEPTH][NH][4];    // V: tokens 16hh + 4kb + r, dims 8c..8c+7
    // LDS-staged FP8: the raw coalesced loads (rows 8 part + lane / 8, bytes
    // 16 (lane % 8) .. +15 of each half), moved into kr / vr by the stage.
    u32x4 kc[STG && !DMA ? DEPTH : 1][NH][NPART], vc[STG && !DMA ? DEPTH : 1][NH][NPART];
    u32x4 qc[DMA ? 1 : DEPTH][NQ];   // compact Q, loaded with a segment's first step (direct paths)
    int   pg[DEPTH][NH];       // power-of-two path: page of each half (wave-uniform)
    int   pgr[PATH == kPageRuns ? DEPTH : 1][NH][NPART];   // small pages: page of each part
    constexpr int LN = PATH == kPageLane ? DEPTH : 1;
    int   plk[LN][NH][NPART], psl[LN][NH][NPART];          // lane path: byte address of the lane holding
                                                           // the row's page entry, slot in the page
    int   pent[LN];                                        // lane path: table entry `first page + lane`
    int   pk[DEPTH][NH], sk[DEPTH][NH];            // per-lane paths: K token's page and slot
    int   pv[DEPTH][NH][NVL], sv[DEPTH][NH][NVL];  // per-lane paths: V tokens' page(s) and slot(s)

    Cursor C, L, T;
    C.seg = seg_begin;
    cursor_load(C, segs);
    L = C;
    T = C;
    const int* t_row = table_row(p, tbl, sid, T.b);
    bool t_more = true, l_more = true;

    // Page lookups of step T into slot s, then advance T.
    auto lookup = [&](int s) {
        if constexpr (PATH == kPagePow2) {
            if (t_more) {
#pragma unroll
                for (int hh = 0; hh < NH; ++hh)
                    pg[s][hh] = load_uniform(t_row, min(T.tok + 16 * hh, T.w - 1) >> page_shift);
            }
        } else if constexpr (PATH == kPageRuns) {
            if (t_more) {
#pragma unroll
                for (int hh = 0; hh < NH; ++hh)
#pragma unroll
                    for (int part = 0; part < NPART; ++part)
                        pgr[s][hh][part] = load_uniform(t_row, min(T.tok + 16 * hh + RPP * part, T.w - 1) >> page_shift);
            }
        } else if constexpr (PATH == kPageLane) {
            // One table read per lane covers the step's pages (at most
            // NG / P + 1 <= 33 entries); each lane then needs the page of the
            // row it loads in each 1 KiB part, fetched from the lane holding
            // it with ds_bpermute at issue time. Like the other per-lane
            // paths, lookups repeat T's last step once it is exhausted, so
            // that every slot issues the same vector loads.
            const int last  = T.w - 1;
            const int first = page_shift >= 0 ? T.tok >> page_shift : T.tok / P;   // wave-uniform choice
            const int lastp = page_shift >= 0 ? last >> page_shift : last / P;
            pent[s] = t_row[min(first + lane, lastp)];
#pragma unroll
            for (int hh = 0; hh < NH; ++hh)
#pragma unroll
                for (int part = 0; part < NPART; ++part) {
                    const int tk = min(T.tok + 16 * hh + RPP * part + lane / CPR, last);
                    const int qk = page_shift >= 0 ? tk >> page_shift : tk / P;
                    plk[s][hh][part] = 4 * (qk - first);
                    psl[s][hh][part] = tk - qk * P;
                }
        } else {
            // Per-lane lookups repeat T's last step once it is exhausted, so
            // that every slot issues the same vector loads.
            const int last = T.w - 1;
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) {
                const int tk = min(T.tok + 16 * hh + c, last);
                const int qk = PATH == kPageQuad ? (tk >> page_shift) : tk / P;
                pk[s][hh] = t_row[qk];
                sk[s][hh] = tk - qk * P;
                if constexpr (PATH == kPageQuad) {
                    // The lane's 4 V tokens share one page (page_size % 4 == 0).
                    const int tv = min(T.tok + 16 * hh + 4 * kb, last & ~3);
                    const int qv = tv >> page_shift;
                    pv[s][hh][0] = t_row[qv];
                    sv[s][hh][0] = tv - qv * P;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int t  = min(T.tok + 16 * hh + 4 * kb + r, last);
                        const int qv = t / P;
                        pv[s][hh][r] = t_row[qv];
                        sv[s][hh][r] = t - qv * P;
                    }
                }
            }
        }
        if (t_more) {
            const int a = cursor_step<NG>(T, segs, seg_end);
            if (__builtin_expect(a != 0, 0)) {
                if (a < 0) t_more = false;
                else t_row = table_row(p, tbl, sid, T.b);
            }
        }
    };

    // K/V loads of step L into slot s (and Q at a segment start), then advance L.
    auto issue = [&](int s) {
        if constexpr (DMA) {
            // The previous step's stage and Q reads have returned before new
            // rows land.
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            wave_lds_sync();
        }
        const bool first = l_more && L.tok == L.t0;
        const __amdgpu_buffer_rsrc_t qrs =
            buffer_rsrc(p.q + (static_cast<size_t>(L.b) * hq + L.h * G) * kHeadDim, first ? 256 * G : 0);
        if constexpr (DMA) {
            // A segment's Q lands in the wave's Q area with its first K / V
            // (lanes past G x 256 B write zeros).
            if (first) {
#pragma unroll
                for (int n = 0; n < NQ; ++n) lds_load16<0>(qrs, &q_lds[wave][64 * n], 16 * (64 * n + lane));
            }
        } else {
#pragma unroll
            for (int n = 0; n < NQ; ++n)
                qc[s][n] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(qrs, 16 * ((64 * n + lane) % (16 * G)), 0, 0));
        }
        if constexpr (PATH == kPagePow2) {
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) {
                const int t  = L.tok + 16 * hh;          // first token of the half
                const int bt = min(t, L.w - 1);          // a token of the sequence (pages stay in range)
                // The page and the valid tokens of the half are wave-uniform:
                // said so, the K/V buffer resources stay in SGPRs (no per-load
                // waterfall loop).
                const int nv = __builtin_amdgcn_readfirstlane(l_more ? max(0, min(16, L.w - t)) : 0);
                const size_t row0 = static_cast<size_t>(__builtin_amdgcn_readfirstlane(pg[s][hh])) * page_bytes +
                                    static_cast<uint32_t>((L.h * P + (bt & (P - 1))) * ROW);
                const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(kbase + row0, nv * ROW);
                const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(vbase + row0, nv * ROW);
                if constexpr (DMA) {
#pragma unroll
                    for (int part = 0; part < NPART; ++part) {
                        const int off = 1024 * part + ROW * (lane / CPR) + dma_chunk[part];
                        lds_load16<kAux<NT>>(krs, stage + hh * HCH + 64 * part, off);
                        lds_load16<kAux<NT>>(vrs, stage + (NH + hh) * HCH + 64 * part, off);
                    }
                    continue;
                } else if constexpr (STG) {
#pragma unroll
                    for (int part = 0; part < NPART; ++part) {
                        kc[s][hh][part] = __builtin_bit_cast(
                            u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, 1024 * part + 16 * lane, 0, kAux<NT>));
                        vc[s][hh][part] = __builtin_bit_cast(
                            u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, 1024 * part + 16 * lane, 0, kAux<NT>));
                    }
                    continue;
                }
#pragma unroll
                for (int u = 0; u < NK; ++u) {
                    if constexpr (KL == 16)
                        kr[s][hh][u] = __builtin_bit_cast(
                            u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, k_lane_off + KSTEP * u, 0, kAux<NT>));
                    else
                        kr[s][hh][u] = __builtin_bit_cast(
                            u32x2, __builtin_amdgcn_raw_buffer_load_b64(krs, k_lane_off + KSTEP * u, 0, kAux<NT>));
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (EB == 2)
                        vr[s][hh][r] = __builtin_bit_cast(
                            u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, v_lane_off + r * ROW, 0, kAux<NT>));
                    else
                        vr[s][hh][r] = __builtin_bit_cast(
                            u32x2, __builtin_amdgcn_raw_buffer_load_b64(vrs, v_lane_off + r * ROW, 0, kAux<NT>));
                }
            }
        } else if constexpr (PATH == kPageRuns) {
#pragma unroll
            for (int hh = 0; hh < NH; ++hh)
#pragma unroll
                for (int part = 0; part < NPART; ++part) {
                    const int t  = L.tok + 16 * hh + RPP * part;   // first token of the part (inside one page)
                    const int bt = min(t, L.w - 1);
                    const int nv = __builtin_amdgcn_readfirstlane(l_more ? max(0, min(RPP, L.w - t)) : 0);
                    const size_t row0 =
                        static_cast<size_t>(__builtin_amdgcn_readfirstlane(pgr[s][hh][part])) * page_bytes +
                        static_cast<uint32_t>((L.h * P + (bt & (P - 1))) * ROW);
                    const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(kbase + row0, nv * ROW);
                    const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(vbase + row0, nv * ROW);
                    if constexpr (DMA) {
                        const int off = ROW * (lane / CPR) + dma_chunk[part];
                        lds_load16<kAux<NT>>(krs, stage + hh * HCH + 64 * part, off);
                        lds_load16<kAux<NT>>(vrs, stage + (NH + hh) * HCH + 64 * part, off);
                    } else {
                        kc[s][hh][part] = __builtin_bit_cast(
                            u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, 16 * lane, 0, kAux<NT>));
                        vc[s][hh][part] = __builtin_bit_cast(
                            u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, 16 * lane, 0, kAux<NT>));
                    }
                }
        } else if constexpr (PATH == kPageLane) {
#pragma unroll
            for (int hh = 0; hh < NH; ++hh)
#pragma unroll
                for (int part = 0; part < NPART; ++part) {
                    const int pgl = __builtin_amdgcn_ds_bpermute(plk[s][hh][part], pent[s]);
                    const size_t row = kv_row_offset<EB>(pgl, L.h, psl[s][hh][part], P, hkv);
                    if constexpr (DMA) {
                        lds_load16<kAux<NT>>(kbase + row + dma_chunk[part], stage + hh * HCH + 64 * part);
                        lds_load16<kAux<NT>>(vbase + row + dma_chunk[part], stage + (NH + hh) * HCH + 64 * part);
                    } else {
                        kc[s][hh][part] = load16<NT>(kbase + row + 16 * (lane % CPR));
                        vc[s][hh][part] = load16<NT>(vbase + row + 16 * (lane % CPR));
                    }
                }
        } else {
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) {
                const unsigned char* kp = kbase + kv_row_offset<EB>(pk[s][hh], L.h, sk[s][hh], P, hkv) + kb * KLANE;
#pragma unroll
                for (int u = 0; u < NK; ++u) {
                    if constexpr (KL == 16) kr[s][hh][u] = load16<NT>(kp + KSTEP * u);
                    else kr[s][hh][u] = load8<NT>(kp + KSTEP * u);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    size_t off;
                    if constexpr (PATH == kPageQuad) {
                        const int tv = min(L.tok + 16 * hh + 4 * kb, (L.w - 1) & ~3);
                        off = kv_row_offset<EB>(pv[s][hh][0], L.h, sv[s][hh][0] + min(r, L.w - 1 - tv), P, hkv);
                    } else {
                        off = kv_row_offset<EB>(pv[s][hh][r], L.h, sv[s][hh][r], P, hkv);
                    }
                    if constexpr (EB == 2) vr[s][hh][r] = load16<NT>(vbase + off + c * VCH);
                    else vr[s][hh][r] = load8<NT>(vbase + off + c * VCH);
                }
            }
        }
        if (l_more && cursor_step<NG>(L, segs, seg_end) < 0) l_more = false;
    };

    // ---- consumer state. m_run = -inf marks a segment start: the first step
    // always takes the rescale path, which then sets the running max (the
    // factor 2^-inf = 0 keeps O = 0 and l = 0).
    u32x4 qf[4];      // B operand of QK MFMA j: Q[head c % G][the dims of K's A operand]
    f32x4 oacc[8];    // O[head 4kb+i][dim 8c+j] = oacc[j][i]
    float m_run = -INFINITY, l_run = 0.f;
    bool  whole = false;
#pragma unroll
    for (int j = 0; j < 8; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto finish_segment = [&]() {
        const int sl = C.seg == seg_begin ? 0 : 1;   // a unit's split segments are its first and last
        float lsum = l_run;
        lsum += __shfl_xor(lsum, 16);
        lsum += __shfl_xor(lsum, 32);
        float m_h[G], inv_h[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            m_h[h]   = readlane_f(m_run, h);
            inv_h[h] = readlane_f(lsum, h);
        }
        if (4 * kb < G) {   // lanes holding live O rows: heads 4kb .. 4kb + HW - 1
            if (whole) {
#pragma unroll
                for (int i = 0; i < HW; ++i) {
                    const float inv = p.v_scale / head_pick<G>(inv_h, kb, i);
                    uint16_t* orow = p.out + (static_cast<size_t>(C.b) * hq + C.h * G + 4 * kb + i) * kHeadDim;
                    u32x4 o;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const f16x2 h2 = {static_cast<_Float16>(oacc[2 * jj][i] * inv),
                                          static_cast<_Float16>(oacc[2 * jj + 1][i] * inv)};
                        o[jj] = __builtin_bit_cast(uint32_t, h2);
                    }
                    *reinterpret_cast<u32x4*>(orow + 8 * c) = o;
                }
            } else {
#pragma unroll
                for (int i = 0; i < HW; ++i) {
                    const float lh  = head_pick<G>(inv_h, kb, i);
                    const float inv = p.v_scale / lh;
                    const float ls  = head_pick<G>(m_h, kb, i) + __log2f(lh);
                    // The LDS and HBM stores stay in separate branches: a pointer
                    // selected between them would be a generic (flat) address.
                    if (merge_here) {
                        float* lrow = &part_lds[2 * wave + sl][(4 * kb + i) * kHeadDim];
                        store_row(lrow, oacc, i, inv, c);
                        if (c == 0) lse_lds[2 * wave + sl][4 * kb + i] = ls;
                    } else {
                        float* prow = p.partial_out + (static_cast<size_t>(C.seg) * G + 4 * kb + i) * kHeadDim;
                        store_row(prow, oacc, i, inv, c);
                        if (c == 0) p.partial_lse[static_cast<size_t>(C.seg) * G + 4 * kb + i] = ls;
                    }
                }
                if (merge_here && lane == 0) {
                    slot_item[wave][sl] = C.b * hkv + C.h;
                    slot_seg[wave][sl]  = C.seg;
                }
            }
        }
        m_run = -INFINITY;
        l_run = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    auto rescale = [&](float xmax) {
        float mx = fmaxf(xmax, __shfl_xor(xmax, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = exp2_fast(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
        float a_h[G];
#pragma unroll
        for (int h = 0; h < G; ++h) a_h[h] = readlane_f(alpha, h);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ai = 4 * kb + i < G ? head_pick<G>(a_h, kb, i) : 1.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) oacc[j][i] *= ai;
        }
    };

    // A step's data into registers: the segment's Q at its first step, and on
    // the stage paths the step's K / V rows out of the LDS stage.
    auto consume_in = [&](int s) {
        if constexpr (DMA) {
            // With one step in flight, every vector memory operation
            // outstanding here belongs to this step: its Q and rows are in
            // LDS once they have all returned.
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            wave_lds_sync();
        }
        if (__builtin_expect(C.tok == C.t0, 0)) {
            // Q of the new segment: compact -> LDS -> B-operand layout.
            u32x4* ql = q_lds[wave];
            if constexpr (!DMA) {
                wave_lds_sync();   // the previous segment's Q reads are done
#pragma unroll
                for (int n = 0; n < NQ; ++n)
                    if (64 * n + lane < 16 * G) ql[64 * n + lane] = qc[s][n];
                wave_lds_sync();   // every lane's Q write lands before any lane reads
            }
            const int hc = c & (G - 1);
#pragma unroll
            for (int j = 0; j < 4; ++j) qf[j] = ql[16 * hc + (KNAT ? 4 * j + kb : 4 * kb + j)];
            const int item = C.b * hkv + C.h;
            whole = isb[item + 1] - isb[item] == 1;
        }
        if constexpr (STG) {
            // Coalesced rows -> LDS (16-byte chunk j of row r at chunk j ^ (r % CPR))
            // -> the K / V lane layouts of the direct loads.
            u32x4* st = stage;
            if constexpr (!DMA) {
                const int wrow = lane / CPR;   // row within a 1 KiB part
                wave_lds_sync();   // the previous step's stage reads are done
#pragma unroll
                for (int hh = 0; hh < NH; ++hh)
#pragma unroll
                    for (int part = 0; part < NPART; ++part) {
                        const int row  = RPP * part + wrow;
                        const int slot = CPR * row + ((lane % CPR) ^ swz(row));
                        st[hh * HCH + slot]        = kc[s][hh][part];
                        st[(NH + hh) * HCH + slot] = vc[s][hh][part];
                    }
                wave_lds_sync();   // every lane's rows land before any lane reads its layout
            }
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) {
#pragma unroll
                for (int u = 0; u < NK; ++u) {
                    const int ch = (kb * KLANE + KSTEP * u) / 16;   // chunk of row c this load holds
                    kr[s][hh][u] = st[hh * HCH + CPR * c + (ch ^ swz(c))];
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 4 * kb + r;
                    const u32x4* vrow = st + (NH + hh) * HCH + CPR * row;
                    if constexpr (EB == 2) {
                        vr[s][hh][r] = vrow[c ^ swz(row)];
                    } else {
                        vr[s][hh][r] = reinterpret_cast<const u32x2*>(vrow)[2 * ((c >> 1) ^ swz(row)) + (c & 1)];
                    }
                }
            }
        }
    };
    // A step's arithmetic on those registers: scores, online softmax, P V, and
    // the segment's output or partial after its last step.
    auto consume_math = [&](int s) {
        // S^T[token][head] per 16-token half; lane (c, kb) gets tokens 4kb+i.
        float x[NH][4];
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
            f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f16x8 a;
                if constexpr (EB == 2) {
                    a = __builtin_bit_cast(f16x8, kr[s][hh][j]);
                } else if constexpr (KNAT) {
                    a = fp8x8_to_f16x8(kr[s][hh][j][0], kr[s][hh][j][1]);
                } else {
                    const KRaw w = kr[s][hh][j >> 1];
                    a = fp8x8_to_f16x8(w[2 * (j & 1)], w[2 * (j & 1) + 1]);
                }
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(f16x8, qf[j]), sacc, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) x[hh][i] = sacc[i] * qk_scale;
        }
        const int lim = C.w - C.tok;   // valid tokens of the step
        if (__builtin_expect(lim < NG, 0)) {
#pragma unroll
            for (int hh = 0; hh < NH; ++hh)
#pragma unroll
                for (int i = 0; i < 4; ++i) x[hh][i] = 16 * hh + 4 * kb + i < lim ? x[hh][i] : -INFINITY;
        }
        float xmax = fmaxf(fmaxf(x[0][0], x[0][1]), fmaxf(x[0][2], x[0][3]));
        if constexpr (NH > 1) xmax = fmaxf(xmax, fmaxf(fmaxf(x[1][0], x[1][1]), fmaxf(x[1][2], x[1][3])));
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(c < G && xmax > m_run + kRescaleSlack) != 0, 0))
            rescale(xmax);
        float pr[NH][4];
        float psum = 0.f;
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
#pragma unroll
            for (int i = 0; i < 4; ++i) pr[hh][i] = exp2_fast(x[hh][i] - m_run);
            psum += (pr[hh][0] + pr[hh][1]) + (pr[hh][2] + pr[hh][3]);
        }
        l_run += psum;

        // O[head][dim] += P[head][token] V[token][dim]; MFMA j covers dims 8c + j.
        if constexpr (NH == 1) {
            const f16x4 pa = {static_cast<_Float16>(pr[0][0]), static_cast<_Float16>(pr[0][1]),
                              static_cast<_Float16>(pr[0][2]), static_cast<_Float16>(pr[0][3])};
            if constexpr (EB == 2) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                    u32x2 bw;
                    bw[0] = __builtin_amdgcn_perm(vr[s][0][1][j >> 1], vr[s][0][0][j >> 1], sel);
                    bw[1] = __builtin_amdgcn_perm(vr[s][0][3][j >> 1], vr[s][0][2][j >> 1], sel);
                    oacc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(f16x4, bw), oacc[j], 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int w = 0; w < 2; ++w) {
                    // bytes [t0 d, t1 d, t0 d+1, t1 d+1] for d = 4w (lo) and 4w+2 (hi)
                    const uint32_t lo01 = __builtin_amdgcn_perm(vr[s][0][1][w], vr[s][0][0][w], 0x05010400u);
                    const uint32_t hi01 = __builtin_amdgcn_perm(vr[s][0][1][w], vr[s][0][0][w], 0x07030602u);
                    const uint32_t lo23 = __builtin_amdgcn_perm(vr[s][0][3][w], vr[s][0][2][w], 0x05010400u);
                    const uint32_t hi23 = __builtin_amdgcn_perm(vr[s][0][3][w], vr[s][0][2][w], 0x07030602u);
                    const u32x2 b0 = {fp8x2_to_f16x2<false>(lo01), fp8x2_to_f16x2<false>(lo23)};
                    const u32x2 b1 = {fp8x2_to_f16x2<true>(lo01), fp8x2_to_f16x2<true>(lo23)};
                    const u32x2 b2 = {fp8x2_to_f16x2<false>(hi01), fp8x2_to_f16x2<false>(hi23)};
                    const u32x2 b3 = {fp8x2_to_f16x2<true>(hi01), fp8x2_to_f16x2<true>(hi23)};
                    oacc[4 * w + 0] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(f16x4, b0), oacc[4 * w + 0], 0, 0, 0);
                    oacc[4 * w + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(f16x4, b1), oacc[4 * w + 1], 0, 0, 0);
                    oacc[4 * w + 2] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(f16x4, b2), oacc[4 * w + 2], 0, 0, 0);
                    oacc[4 * w + 3] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(f16x4, b3), oacc[4 * w + 3], 0, 0, 0);
                }
            }
        } else {
            // One 32-token k-block: k-index 8kb + i <-> token 4kb + i of half 0
            // (i < 4) and token 16 + 4kb + (i - 4) of half 1.
            const f16x8 pa = {static_cast<_Float16>(pr[0][0]), static_cast<_Float16>(pr[0][1]),
                              static_cast<_Float16>(pr[0][2]), static_cast<_Float16>(pr[0][3]),
                              static_cast<_Float16>(pr[1][0]), static_cast<_Float16>(pr[1][1]),
                              static_cast<_Float16>(pr[1][2]), static_cast<_Float16>(pr[1][3])};
            if constexpr (EB == 2) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                    const int d = j >> 1;
                    u32x4 bw;
                    bw[0] = __builtin_amdgcn_perm(vr[s][0][1][d], vr[s][0][0][d], sel);
                    bw[1] = __builtin_amdgcn_perm(vr[s][0][3][d], vr[s][0][2][d], sel);
                    bw[2] = __builtin_amdgcn_perm(vr[s][1][1][d], vr[s][1][0][d], sel);
                    bw[3] = __builtin_amdgcn_perm(vr[s][1][3][d], vr[s][1][2][d], sel);
                    oacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, __builtin_bit_cast(f16x8, bw), oacc[j], 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int w = 0; w < 2; ++w) {
                    uint32_t lo01[2], hi01[2], lo23[2], hi23[2];
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        lo01[hh] = __builtin_amdgcn_perm(vr[s][hh][1][w], vr[s][hh][0][w], 0x05010400u);
                        hi01[hh] = __builtin_amdgcn_perm(vr[s][hh][1][w], vr[s][hh][0][w], 0x07030602u);
                        lo23[hh] = __builtin_amdgcn_perm(vr[s][hh][3][w], vr[s][hh][2][w], 0x05010400u);
                        hi23[hh] = __builtin_amdgcn_perm(vr[s][hh][3][w], vr[s][hh][2][w], 0x07030602u);
                    }
                    const u32x4 b0 = {fp8x2_to_f16x2<false>(lo01[0]), fp8x2_to_f16x2<false>(lo23[0]),
                                      fp8x2_to_f16x2<false>(lo01[1]), fp8x2_to_f16x2<false>(lo23[1])};
                    const u32x4 b1 = {fp8x2_to_f16x2<true>(lo01[0]), fp8x2_to_f16x2<true>(lo23[0]),
                                      fp8x2_to_f16x2<true>(lo01[1]), fp8x2_to_f16x2<true>(lo23[1])};
                    const u32x4 b2 = {fp8x2_to_f16x2<false>(hi01[0]), fp8x2_to_f16x2<false>(hi23[0]),
                                      fp8x2_to_f16x2<false>(hi01[1]), fp8x2_to_f16x2<false>(hi23[1])};
                    const u32x4 b3 = {fp8x2_to_f16x2<true>(hi01[0]), fp8x2_to_f16x2<true>(hi23[0]),
                                      fp8x2_to_f16x2<true>(hi01[1]), fp8x2_to_f16x2<true>(hi23[1])};
                    oacc[4 * w + 0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, __builtin_bit_cast(f16x8, b0), oacc[4 * w + 0], 0, 0, 0);
                    oacc[4 * w + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, __builtin_bit_cast(f16x8, b1), oacc[4 * w + 1], 0, 0, 0);
                    oacc[4 * w + 2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, __builtin_bit_cast(f16x8, b2), oacc[4 * w + 2], 0, 0, 0);
                    oacc[4 * w + 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, __builtin_bit_cast(f16x8, b3), oacc[4 * w + 3], 0, 0, 0);
                }
            }
        }
        if (__builtin_expect(C.tok + NG >= C.w, 0)) finish_segment();
    };

    // ---- prologue: pages of steps 0..DEPTH-1, then their loads, each
    // followed by the pages DEPTH steps further on.
#pragma unroll
    for (int s = 0; s < DEPTH; ++s) lookup(s);
#pragma unroll
    for (int s = 0; s < DEPTH; ++s) {
        issue(s);
        lookup(s);
    }

    // ---- steady state: consume step k, refill its slot with step k + DEPTH.
    // Each exit leaves the loop directly (a flag tested at the loop head would
    // give the compiler a path from the exit back into the loop, over which
    // it cannot count the outstanding loads and waits for all of them).
    static_assert(DEPTH >= 1 && DEPTH <= 4, "ring of 1 to 4 slots");
    auto advance = [&](int s) {
        consume_in(s);
        if constexpr (DMA) {
            // The stage is in registers: the next step's rows land in it while
            // this step's arithmetic runs (past the last step the loads are
            // empty).
            issue(s);
            lookup(s);
        }
        consume_math(s);
        if (cursor_step<NG>(C, segs, seg_end) < 0) return false;
        if constexpr (!DMA) {
            issue(s);
            lookup(s);
        }
        return true;
    };
    for (;;) {
        if (!advance(0)) break;
        if constexpr (DEPTH > 1) if (!advance(1)) break;
        if constexpr (DEPTH > 2) if (!advance(2)) break;
        if constexpr (DEPTH > 3) if (!advance(3)) break;
    }
    }   // seg_begin < seg_end
    stamp(1 + wave);
    if (wave == 0) stamp_clock(21);

    if (merge_here) {
        __syncthreads();
        block_merge<G>(p, isb, slot_item, slot_seg, part_lds, lse_lds, last_lds, threadIdx.x, lblock);
    }
}

// The kernels: one per element width, each with its own register budget. The
// block table, the slot ids and the plan's segment and row arrays, which the
// kernels only read, also come as separate __restrict__ arguments: through the
// params struct's pointers the compiler cannot tell them from the output, so
// inside the loop it read them with vector loads; as restrict arguments they
// are scalar loads (out of the vector memory counters and the VGPRs: 8 fewer
// VGPRs in the FP8 kernel, 10 fewer on the per-lane page path). They come
// first, with the unit count, ahead of the params struct: the library is built
// with kernel-argument preloading, which places the arguments before the
// first struct passed by value in SGPRs when a wave starts, so a wave's first
// load (its unit's segment range) does not wait for a read of the argument
// segment (0.15 us per launch on every config).
template <int G, int NG, int DEPTH, int PATH>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(PA_FP16_WAVES_PER_EU)))
void decode_split_kernel_f16(const int32_t* __restrict__ cta, const int32_t* __restrict__ segp,
                             const int32_t* __restrict__ tbl, const int32_t* __restrict__ sid, int num_units,
                             int page_shift, const int32_t* __restrict__ isb, const pa_decode_params p) {
    decode_split_body<2, G, NG, DEPTH, PATH>(p, cta, num_units, page_shift, tbl, sid, segp, isb);
}

template <int G, int NG, int DEPTH, int PATH>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(PA_FP8_WAVES_PER_EU)))
void decode_split_kernel_fp8(const int32_t* __restrict__ cta, const int32_t* __restrict__ segp,
                             const int32_t* __restrict__ tbl, const int32_t* __restrict__ sid, int num_units,
                             int page_shift, const int32_t* __restrict__ isb, const pa_decode_params p) {
    decode_split_body<1, G, NG, DEPTH, PATH>(p, cta, num_units, page_shift, tbl, sid, segp, isb);
}

// ---------------------------------------------------------------------------
// Merge (decode_kernels.cuh:409-432): one block per (query head, batch row,
// DS-dim slice) of a row split over n > 1 segments; slicing the 128 dims over
// 128 / DS blocks spreads a few long rows (one 131072-token sequence: 32
// (query head, row) pairs of 256 segments) over
// every CU, since one CU streams only ~25 GB/s. DS / 4 lanes cover a segment's
// slice (4 dims each, one 16-byte load), so a wave covers 256 / DS segments at
// a time. A single pass over the segments with a running base-2 maximum per
// lane (no separate pass for the maximum: one dependent round trip fewer);
// lanes of the same dims combine by shuffles, waves in LDS.
//
// The arrays it reads first come ahead of the params struct, preloaded in SGPRs
// (as for the split kernels).
template <int G, int WAVES, int DS>
__global__ __launch_bounds__(64 * WAVES) void decode_merge_kernel(const int32_t* __restrict__ isb,
                                                                  const float* __restrict__ part_out,
                                                                  const float* __restrict__ part_lse,
                                                                  int num_kv_heads, const pa_decode_params p) {
    constexpr int LPS = DS / 4;      // lanes per segment
    constexpr int SPW = 64 / LPS;    // segments per wave per pass
    // The combine below exchanges lanes 4, 8, 16 and 32 apart only.
    static_assert(LPS >= 4 && LPS <= 32 && (LPS & (LPS - 1)) == 0, "dim slices of 16, 32, 64 or 128");
    const int hqi  = blockIdx.x;
    const int b    = blockIdx.y;
    const int d0   = blockIdx.z * DS;
    const int item = b * num_kv_heads + hqi / G;
    const int g    = hqi % G;
    const int s0 = isb[item];
    const int n  = isb[item + 1] - s0;
    if (n <= 1) return;

    __shared__ float4 acc_lds[WAVES][LPS];
    __shared__ float  den_lds[WAVES], max_lds[WAVES];

    const int t    = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;

    // One pass: each lane keeps its own running maximum m of the base-2 LSEs
    // it has seen and sum_s 2^(lse_s - m) o_s, sum_s 2^(lse_s - m), rescaled
    // when m grows (an empty lane keeps m = -inf and contributes 0).
    const int dq = lane % LPS;       // which 4 dims of the slice
    const int sl = lane / LPS;       // which segment of the wave's pass
    float4 acc = {0.f, 0.f, 0.f, 0.f};
    float  den = 0.f, m = -INFINITY;
#pragma unroll 4
    for (int i = wave * SPW + sl; i < n; i += WAVES * SPW) {
        const size_t sg  = static_cast<size_t>(s0 + i);
        const float  lse = part_lse[sg * G + g];
        const float4 o   = *reinterpret_cast<const float4*>(part_out + (sg * G + g) * kHeadDim + d0 + 4 * dq);
        const float  mn  = fmaxf(m, lse);
        const float  f   = exp2_fast(m - mn);      // 0 while m = -inf
        const float  wgt = exp2_fast(lse - mn);
        acc.x = fmaf(wgt, o.x, acc.x * f);
        acc.y = fmaf(wgt, o.y, acc.y * f);
        acc.z = fmaf(wgt, o.z, acc.z * f);
        acc.w = fmaf(wgt, o.w, acc.w * f);
        den   = fmaf(den, f, wgt);
        m     = mn;
    }
    // Combine (m, den, acc) states: lanes of the same dims, then waves. The
    // partner state comes without an LDS round trip: within a row of 16
    // lanes from a DPP rotation by o (rotations by 4 and then 8 combine the
    // same four lanes as exchanges with lanes 4 and 8 apart), across rows
    // from gfx950's row / half swaps (v_permlane16_swap, v_permlane32_swap:
    // with the value as both operands, the first result holds lane i - o in
    // the upper row / half, the second lane i + o in the lower one).
    auto scale_to = [](float mi, float mt) { return mi == -INFINITY ? 0.f : exp2_fast(mi - mt); };
    auto partner = [lane](float x, int o) {
        const unsigned u = __builtin_bit_cast(unsigned, x);
        if (o == 4) return dpp_f32<0x124>(x);   // row_ror:4
        if (o == 8) return dpp_f32<0x128>(x);   // row_ror:8
        if (o == 16) {
            const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
            return __builtin_bit_cast(float, (lane & 16) ? r[0] : r[1]);
        }
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return __builtin_bit_cast(float, (lane & 32) ? r[0] : r[1]);
    };
#pragma unroll
    for (int o = LPS; o < 64; o <<= 1) {
        const float m2 = partner(m, o);
        const float mt = fmaxf(m, m2);
        const float f1 = scale_to(m, mt), f2 = scale_to(m2, mt);
        acc.x = acc.x * f1 + partner(acc.x, o) * f2;
        acc.y = acc.y * f1 + partner(acc.y, o) * f2;
        acc.z = acc.z * f1 + partner(acc.z, o) * f2;
        acc.w = acc.w * f1 + partner(acc.w, o) * f2;
        den   = den * f1 + partner(den, o) * f2;
        m     = mt;
    }
    if (lane < LPS) acc_lds[wave][lane] = acc;
    if (lane == 0) {
        den_lds[wave] = den;
        max_lds[wave] = m;
    }
    __syncthreads();
    if (wave == 0 && lane < LPS) {
        float mt = max_lds[0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) mt = fmaxf(mt, max_lds[w]);
        float4 a = {0.f, 0.f, 0.f, 0.f};
        float  d = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float f = scale_to(max_lds[w], mt);
            a.x = fmaf(acc_lds[w][lane].x, f, a.x);
            a.y = fmaf(acc_lds[w][lane].y, f, a.y);
            a.z = fmaf(acc_lds[w][lane].z, f, a.z);
            a.w = fmaf(acc_lds[w][lane].w, f, a.w);
            d   = fmaf(den_lds[w], f, d);
        }
        const f16x2 lo = {static_cast<_Float16>(a.x / d), static_cast<_Float16>(a.y / d)};
        const f16x2 hi = {static_cast<_Float16>(a.z / d), static_cast<_Float16>(a.w / d)};
        *reinterpret_cast<u32x2*>(p.out + (static_cast<size_t>(b) * p.num_q_heads + hqi) * kHeadDim + d0 + 4 * dq) =
            u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
    }
}

// ---------------------------------------------------------------------------
// Dispatch.

// Steps in flight on the per-lane page paths (they keep the power-of-two
// path's step, so results do not depend on the page size): kPageLane, and
// kPageQuad / kPageAny in FP8 builds without the LDS stage.
#ifndef PA_FP16_LANE_DEPTH
#define PA_FP16_LANE_DEPTH 1
#endif
#ifndef PA_FP8_LANE_DEPTH
#define PA_FP8_LANE_DEPTH 2
#endif
template <int EB> constexpr int kLaneDepth = kLdsDma ? 1 : EB == 2 ? PA_FP16_LANE_DEPTH : PA_FP8_LANE_DEPTH;
// Steps in flight on the power-of-two path (one when it is staged through
// LDS-destination loads) and on the staged small-page path.
template <int EB> constexpr int kPow2Depth = kLdsDma && Tune<EB>::stage ? 1 : Tune<EB>::depth;
template <int EB> constexpr int kRunsDepth = kLdsDma ? 1 : Tune<EB>::depth;

template <int EB, int G, int NG, int DEPTH, int PATH>
hipError_t launch_split_p(const pa_decode_params& p, int shift, hipStream_t s) {
    const int blocks = (p.num_ctas + kWaves - 1) / kWaves;
    if constexpr (EB == 2)
        hipLaunchKernelGGL((decode_split_kernel_f16<G, NG, DEPTH, PATH>), dim3(blocks), dim3(64 * kWaves), 0, s,
                           p.cta_seg_begin, p.segments, p.block_table, p.slot_ids, p.num_ctas, shift,
                           p.item_seg_begin, p);
    else
        hipLaunchKernelGGL((decode_split_kernel_fp8<G, NG, DEPTH, PATH>), dim3(blocks), dim3(64 * kWaves), 0, s,
                           p.cta_seg_begin, p.segments, p.block_table, p.slot_ids, p.num_ctas, shift,
                           p.item_seg_begin, p);
    return hipGetLastError();
}

template <int EB, int G>
hipError_t launch_split_g(const pa_decode_params& p, hipStream_t s) {
    const int  P     = p.page_size;
    const bool pow2  = (P & (P - 1)) == 0;
    const int  shift = pow2 ? __builtin_ctz(static_cast<unsigned>(P)) : 0;
    if (pow2 && P >= 16) {
        // Byte offsets of one page and of one (kv head, slot) inside it are 32-bit.
        if (static_cast<long long>(p.num_kv_heads) * P * kRowBytes<EB> >= (1ll << 31))
            throw std::invalid_argument("decode: page_size * num_kv_heads * row bytes must be below 2^31");
        return launch_split_p<EB, G, Tune<EB>::step, kPow2Depth<EB>, kPagePow2>(p, shift, s);
    }
    if constexpr (EB == 2 || Tune<EB>::stage) {
        // Pages of whole 1 KiB parts (4 fp16 rows, 8 FP8 rows) through the LDS stage.
        if (P == 8 || (EB == 2 && P == 4)) {
            if (static_cast<long long>(p.num_kv_heads) * P * kRowBytes<EB> >= (1ll << 31))
                throw std::invalid_argument("decode: page_size * num_kv_heads * row bytes must be below 2^31");
            return launch_split_p<EB, G, Tune<EB>::step, kRunsDepth<EB>, kPageRuns>(p, shift, s);
        }
        // Any other size: per-lane rows through the LDS stage (shift -1: divide).
        return launch_split_p<EB, G, Tune<EB>::step, kLaneDepth<EB>, kPageLane>(p, pow2 ? shift : -1, s);
    } else {
        if (pow2 && P >= 4) return launch_split_p<EB, G, Tune<EB>::step, kLaneDepth<EB>, kPageQuad>(p, shift, s);
        return launch_split_p<EB, G, Tune<EB>::step, kLaneDepth<EB>, kPageAny>(p, shift, s);
    }
}

template <int EB>
hipError_t launch_split_e(const pa_decode_params& p, int group, hipStream_t s) {
    switch (group) {
        case 1: return launch_split_g<EB, 1>(p, s);
        case 2: return launch_split_g<EB, 2>(p, s);
        case 4: return launch_split_g<EB, 4>(p, s);
        case 8: return launch_split_g<EB, 8>(p, s);
    }
    throw std::invalid_argument("unsupported GQA group size " + std::to_string(group));
}

// About four segments per lane measured best (4 x 1024 tokens: 64 segments
// per row, one wave; 1 x 131072: 256, four waves); sixteen waves per block
// cost ~1 us more at 1 x 131072.
template <int G, int DS>
hipError_t launch_merge_gd(const pa_decode_params& p, hipStream_t s) {
    const dim3 grid(p.num_q_heads, p.batch, kHeadDim / DS);
    constexpr int SPW = 256 / DS;    // segments one wave covers per pass
    const int m = p.max_item_segments;
    if (m > 0 && m <= 4 * SPW)
        hipLaunchKernelGGL((decode_merge_kernel<G, 1, DS>), grid, dim3(64), 0, s, p.item_seg_begin, p.partial_out,
                           p.partial_lse, p.num_kv_heads, p);
    else
        hipLaunchKernelGGL((decode_merge_kernel<G, 4, DS>), grid, dim3(256), 0, s, p.item_seg_begin, p.partial_out,
                           p.partial_lse, p.num_kv_heads, p);
    return hipGetLastError();
}

// Dim slices per (head, row): enough blocks to reach every CU when few rows
// are split (at least ~1024 blocks), whole rows when many are.
template <int G>
hipError_t launch_merge_g(const pa_decode_params& p, hipStream_t s) {
    const long pairs = static_cast<long>(p.batch) * p.num_q_heads;
    if (pairs >= 1024) return launch_merge_gd<G, 128>(p, s);
    if (pairs >= 512) return launch_merge_gd<G, 64>(p, s);
    if (pairs >= 256) return launch_merge_gd<G, 32>(p, s);
    return launch_merge_gd<G, 16>(p, s);
}

int checked_group(const pa_decode_params& p) {
    if (p.head_dim != kHeadDim) throw std::invalid_argument("unsupported head_dim " + std::to_string(p.head_dim));
    if (p.num_kv_heads <= 0 || p.num_q_heads % p.num_kv_heads != 0)
        throw std::invalid_argument("num_q_heads must be a multiple of num_kv_heads");
    const int g = p.num_q_heads / p.num_kv_heads;
    if (g != 1 && g != 2 && g != 4 && g != 8)
        throw std::invalid_argument("unsupported GQA group size " + std::to_string(g));
    return g;
}

template <int EB, int G>
const void* split_symbol() {
    if constexpr (EB == 2)
        return reinterpret_cast<const void*>(
            &decode_split_kernel_f16<G, Tune<EB>::step, kPow2Depth<EB>, kPagePow2>);
    else
        return reinterpret_cast<const void*>(
            &decode_split_kernel_fp8<G, Tune<EB>::step, kPow2Depth<EB>, kPagePow2>);
}

}  // namespace

int kernel_tile_tokens(int dtype, int group) {
    check_kv_dtype(dtype);
    if (group != 1 && group != 2 && group != 4 && group != 8)
        throw std::invalid_argument("unsupported GQA group size " + std::to_string(group));
    return dtype == PA_KV_FP16 ? Tune<2>::step : Tune<1>::step;
}

int kernel_units_per_cu(int dtype, int group) {
    check_kv_dtype(dtype);
    const void* fn = nullptr;
    const bool fp16 = dtype == PA_KV_FP16;
    switch (group) {
        case 1: fn = fp16 ? split_symbol<2, 1>() : split_symbol<1, 1>(); break;
        case 2: fn = fp16 ? split_symbol<2, 2>() : split_symbol<1, 2>(); break;
        case 4: fn = fp16 ? split_symbol<2, 4>() : split_symbol<1, 4>(); break;
        case 8: fn = fp16 ? split_symbol<2, 8>() : split_symbol<1, 8>(); break;
        default: throw std::invalid_argument("unsupported GQA group size " + std::to_string(group));
    }
    int blocks = 0;
    hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, 64 * kWaves, 0),
              "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    // At most the waves per SIMD the kernel is tuned for (4 SIMDs per CU): a
    // build that happens to fit more (fewer registers) keeps the measured
    // best grid, since more concurrent streams per CU read HBM less
    // efficiently.
    const int tuned = 4 * (fp16 ? PA_FP16_WAVES_PER_EU : PA_FP8_WAVES_PER_EU) / kWaves;
    return std::max(1, std::min(blocks, tuned)) * kWaves;
}

// A plan's split rows are merged either by the merge kernel (needs_merge) or
// inside the split kernel (block_merge), never both: with block_merge the
// workspace holds partial rows only at the slots the split kernel merges
// through, and the merge kernel would read the others unwritten.
void check_merge_fields(const pa_decode_params& p) {
    if (p.needs_merge && p.block_merge)
        throw std::invalid_argument("decode: needs_merge and block_merge exclude each other (bind sets them)");
}

hipError_t launch_decode_split(int dtype, const pa_decode_params& p, hipStream_t s) {
    check_kv_dtype(dtype);
    const int g = checked_group(p);
    check_merge_fields(p);
    if (p.num_ctas <= 0) return hipSuccess;
    if (p.page_size <= 0 || p.block_table_stride <= 0 || p.batch <= 0)
        throw std::invalid_argument("decode: page_size, block_table_stride and batch must be positive");
    if (!p.q || !p.out || !p.k_cache || !p.v_cache || !p.block_table || !p.segments || !p.cta_seg_begin ||
        !p.item_seg_begin)
        throw std::invalid_argument("decode: null pointer in params");
    if ((p.needs_merge || p.block_merge) && (!p.partial_out || !p.partial_lse))
        throw std::invalid_argument("decode: split rows need the partial workspace");
    if (p.block_merge < 0 || p.block_merge > 2) throw std::invalid_argument("decode: block_merge must be 0, 1 or 2");
    if (p.block_merge == 2 && !p.merge_counters)
        throw std::invalid_argument("decode: block_merge 2 needs the plan's merge counters");
    return dtype == PA_KV_FP16 ? launch_split_e<2>(p, g, s) : launch_split_e<1>(p, g, s);
}

hipError_t launch_decode_merge(int dtype, const pa_decode_params& p, hipStream_t s) {
    check_kv_dtype(dtype);
    const int g = checked_group(p);
    check_merge_fields(p);
    if (!p.needs_merge || p.batch <= 0) return hipSuccess;
    if (!p.partial_out || !p.partial_lse || !p.item_seg_begin || !p.out)
        throw std::invalid_argument("decode merge: null pointer in params");
    switch (g) {
        case 1: return launch_merge_g<1>(p, s);
        case 2: return launch_merge_g<2>(p, s);
        case 4: return launch_merge_g<4>(p, s);
        case 8: return launch_merge_g<8>(p, s);
    }
    return hipSuccess;
}

}  // namespace pa
