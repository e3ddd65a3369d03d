// Kernel templates of the MXFP4 A4W4 GEMM and their launchers.  Included by
// gemm_a4w4.hip (host side: configurations, planner, C ABI), which declares
// the launcher instantiations extern, and by the gemm_inst_*.hip files, which
// instantiate them: the kernel families compile as separate translation
// units, in parallel.
#pragma once

#include <type_traits>

#include "mxfp4_device.h"
#include "mbs_gemm_a4w4.h"

namespace mbs {

// One copy per translation unit (each instantiation file is its own code object).
static __constant__ FactorTable kFactors = FactorTable();

__device__ __forceinline__ float factor_of(uint32_t b)
{
    return __uint_as_float(kFactors.bits[b & 255]);
}

struct GemmArgs {
    const uint8_t* A;
    const uint8_t* B;
    const uint8_t* As;
    const uint8_t* Bs;
    const uint8_t* Af;  // nullable (both or neither)
    const uint8_t* Bf;
    uint16_t* out;      // bf16 [Mpad, N]
    float* ws;          // split-K partials [splits][M][N] fp32, or null
    int M, N, K, snp;   // snp = scaleN_pad
    int tiles_m, tiles_n;
    int splits, sps;    // K-splits and 128-K stages per split (even)
    // Grouped (MoE) GEMM: expert e owns rows [groups[e], groups[e+1]) of A
    // (multiples of 32) and the e-th [N, K/2] block of B, its scales and
    // factors.  Null for a dense GEMM.
    const int* groups;
    int n_groups;
    // Epilogue: out = bf16(acc * (alpha * f(a) * f(b)) + bias[n]); alpha 1 and
    // no bias leave the plain product.  bias: bf16 [N] (grouped: [E][N]) or null.
    float alpha;
    const uint16_t* bias;
    // Phase-timer sums (kPhSlots words; timer builds only, else null).
    unsigned long long* phase;
};
// Most experts a grouped launch takes (the per-expert tile table lives in LDS).
constexpr int kMaxGroups = 1024;

// ---------------------------------------------------------------------------
// Phase timer of the persistent kernel (built only with MBS_PHASE_TIMER=1,
// into a separate library; the product build compiles every call below to
// nothing).  Each wave stamps the shader clock (s_memtime) at the phase
// boundaries of its loop and sums the intervals per phase in SGPRs; at the
// end lane 0 adds them into GemmArgs::phase with vector atomics:
//   [kPhPro]   kernel start -> first stage,
//   [kPhWait]  stage-top vmcnt waits (and the one before each epilogue),
//   [kPhBar]   the workgroup barriers that follow them,
//   [kPhBody]  stage bodies: MFMAs, LDS reads and the loads they issue,
//   [kPhEpi]   MFMA drain and epilogue (conversion, lane swaps, stores),
//   [kPhNext]  the next unit's set-up (factor and bias DMAs, unit and
//              offset arithmetic) up to its first stage,
//   [kPhStages], [kPhUnits]  stage and unit counts,
// (per workgroup: GemmArgs::phase holds gridDim.x x kPhSlots words)
//   [kPhClk], [kPhRt]  s_memtime and s_memrealtime (100 MHz) ticks of the
//              whole kernel, wave 0 of each workgroup: their ratio is the
//              shader clock the kernel ran at.
// The stamps' s_waitcnt lgkmcnt(0) also waits for the look-ahead LDS reads
// in flight at a stage top, so the timed kernel runs slightly slower.
#ifndef MBS_PHASE_TIMER
#define MBS_PHASE_TIMER 0
#endif
enum PhaseSlot { kPhPro = 0, kPhWait, kPhBar, kPhBody, kPhEpi, kPhNext, kPhStages, kPhUnits, kPhClk, kPhRt, kPhSlots };

struct PhaseClock {
#if MBS_PHASE_TIMER
    uint64_t last = 0, t0 = 0, r0 = 0;
    uint64_t acc[kPhStages] = {};
    uint32_t stages = 0, units = 0;
    __device__ __forceinline__ void start()
    {
        r0 = __builtin_amdgcn_s_memrealtime();
        t0 = last = __builtin_amdgcn_s_memtime();
    }
    // The time since the previous stamp goes to phase `ph`.
    __device__ __forceinline__ void mark(int ph)
    {
        const uint64_t t = __builtin_amdgcn_s_memtime();
        const uint64_t d = t - last;
        last = t;
        static_for<kPhStages>([&](auto P) { acc[P] += (P == ph) ? d : 0; });
    }
    __device__ __forceinline__ void stage() { ++stages; }
    __device__ __forceinline__ void unit() { ++units; }
    // Each workgroup adds into its own kPhSlots words (out + blockIdx.x *
    // kPhSlots): only its waves contend for them.
    __device__ __forceinline__ void flush(unsigned long long* out)
    {
        const uint64_t t1 = __builtin_amdgcn_s_memtime();
        const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
        if (!out || (threadIdx.x & 63) != 0) return;
        out += (size_t)blockIdx.x * kPhSlots;
        static_for<kPhStages>([&](auto P) { atomicAdd(out + P, (unsigned long long)acc[P]); });
        atomicAdd(out + kPhStages, (unsigned long long)stages);
        atomicAdd(out + kPhUnits, (unsigned long long)units);
        if (threadIdx.x == 0) {
            atomicAdd(out + kPhClk, (unsigned long long)(t1 - t0));
            atomicAdd(out + kPhRt, (unsigned long long)(r1 - r0));
        }
    }
#else
    __device__ __forceinline__ void start() {}
    __device__ __forceinline__ void mark(int) {}
    __device__ __forceinline__ void stage() {}
    __device__ __forceinline__ void unit() {}
    __device__ __forceinline__ void flush(unsigned long long*) {}
#endif
};

// Whether the bf16 epilogue has anything beyond the plain conversion.
inline bool affine_epilogue(const GemmArgs& a)
{
    return (a.Af != nullptr && a.Bf != nullptr) || a.bias != nullptr || a.alpha != 1.0f;
}
// Epilogue form of a launch: 0 plain, 1 factors / alpha, 2 also a bias.
inline int epilogue_form(const GemmArgs& a)
{
    return a.bias != nullptr ? 2 : affine_epilogue(a) ? 1 : 0;
}

// ======================================================================
// B-direct persistent kernel
// ======================================================================
// A workgroup of WGM x WGN waves computes BM x BN tiles.  Only A goes through
// LDS: the preshuffled B is already in MFMA fragment order (one 1-KiB
// contiguous block per 16 rows x 128 K), so each wave loads its B fragments
// with plain 16-byte buffer loads straight into VGPRs, three stages ahead,
// into a 4-deep register ring.  This halves the LDS traffic of the stage
// (LDS bandwidth, not the MFMA pipe, is what limits the all-LDS design).
// A moves through LDS in 256-K "pairs" (two 128-K stages, 128 bytes of each
// row: whole cache lines, so every DMA instruction fetches 8 full lines
// instead of 16 half lines), in a ring of three pair slots; each slot row is
// 8 16-byte chunks stored XOR-swizzled so that the MFMA fragment reads are
// bank-conflict free.  The epilogue turns each pair of 16-column fragments
// into 16-byte row segments with two rounds of permlane swaps.
// M32: the tile runs v_mfma_scale_f32_32x32x64_f8f6f4 (32 x 32 outputs per
// MFMA, 64 K) instead of the 16x16x128 form.  A stage then still reads FM
// A fragments of 1 KiB and loads FN B fragments of 1 KiB, but a fragment
// "row" c of the stage is (K step s = c / FM32, 32-row block c32 = c %
// FM32) and carries FN/2 MFMAs (one per 32-column block).  It covers 1x4
// tiles with 64- or 96-column wave tiles, without K tails, K splits or groups.
template <int BM_, int BN_, int WGM_, int WGN_, bool M32_ = false>
struct BdShape {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_;
    static constexpr bool M32 = M32_;
    static constexpr int NW = WGM * WGN, NT = 64 * NW;
    static constexpr int WM = BM / WGM, WN = BN / WGN;
    static constexpr int FM = WM / 16, FN = WN / 16;    // A fragment reads, B fragment loads per stage
    static constexpr int FM32 = WM / 32, FN32 = WN / 32;
    static constexpr int RW = M32 ? FN / 2 : FN;        // MFMAs per fragment row
    static constexpr int AR = M32 ? FM32 : FM, AC = M32 ? FN32 : FN;   // accumulator blocks
    static_assert(!M32 || (WGM == 1 && (WN == 64 || WN == 96)), "M32 tiles: 1xN waves, 64 or 96 columns per wave");
    static constexpr int AF = BM / 16;                  // A fragments per stage
    // A DMAs per stage: half a pair (BM/2 rows x 128 bytes, 8 rows each),
    // DA per wave.
    static constexpr int DA = (AF + NW - 1) / NW;
    // ADEAL: AF is not a multiple of the wave count but 2 AF is (96 rows: 12
    // DMAs per pair over 4 waves).  The pair's DMAs are then dealt DAP per
    // wave (rows 8 DAP w .. of the slot), DAE of them on its even stage and
    // DAO on the odd one, instead of DA per half with fillers.
    static constexpr bool ADEAL = (AF % NW != 0) && ((2 * AF) % NW == 0);
    static constexpr int DAP = ADEAL ? 2 * AF / NW : 2 * DA;
    static constexpr int DAE = ADEAL ? (DAP + 1) / 2 : DA, DAO = ADEAL ? DAP / 2 : DA;
    static constexpr int NVA = ADEAL ? DAP : DA;        // per-lane A DMA offsets kept
    // scale dwords read per wave per 256-K group: one per 32 rows / columns
    // (16x16x128), two per 32 rows / columns (32x32x64: combined by v_perm)
    static constexpr int SA = M32 ? FM : FM / 2, SB = M32 ? FN : FN / 2;
    static constexpr int PSLOT = BM * 128;              // bytes of one A pair slot
    // Scales of a 256-K group: one 256-byte chunk per 32 rows (A) or columns
    // (B), gathered four chunks per 16-byte LDS DMA.
    static constexpr int CA = BM / 32, CB = BN / 32;
    static constexpr int NSDA = (CA + 3) / 4, NSDB = (CB + 3) / 4, NSD = NSDA + NSDB;
    static constexpr int NSDW = (NSD + NW - 1) / NW;    // scale DMAs per wave per group
    static constexpr int SBUF = NSD * 1024;             // bytes of one scale buffer
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32");
    // MBS factor bytes of a unit in LDS: A rows at [0, 256), B columns in
    // NBC chunks of 256 after them.
    static constexpr int NBC = (BN + 255) / 256;
    static constexpr int FBW = 256 * (1 + NBC);
    // Epilogue bias of a unit in LDS: NBB chunks of 128 bf16 columns, one
    // 256-byte DMA each, FBB per wave.
    static constexpr int NBB = (BN + 127) / 128;
    static constexpr int FBB = (NBB + NW - 1) / NW;
    static_assert(BM <= 256, "one 256-byte chunk of A factor bytes");
    static_assert(NW == 1 ? NBC == 1 : NW >= 1 + NBC, "one factor DMA per wave");
    static_assert(BM % 16 == 0, "pair halves of whole 8-row DMA groups");
    // A pair slots: four where they fit (96-192 rows, 256+ columns), three
    // otherwise.  With four, a slot's previous pair was last read three
    // stages before the DMA that rewrites it (the barrier of the odd stage
    // in between covers it), so even stages wait without a barrier.
    static constexpr int NSLOT = (BM >= 96 && BM <= 192 && BN >= 256) ? 4 : 3;
    static_assert(NSLOT * PSLOT + 2 * SBUF <= 150 * 1024, "LDS budget");
    // Epilogue stores staged through LDS (whole rows per neighbouring lanes)
    // for tiles of 96+ rows; the 64-row tiles, whose short epilogues run with
    // 2-4 workgroups per CU, store straight from registers (the staged form
    // measured 0.7-4% slower there).
    static constexpr bool STAGE_EPI = BM >= 96;
    // epilogue staging bytes per wave: 16 rows (16x16x128) or 32 rows
    // (32x32x64) of one 128-byte line
    static constexpr int EPI_STAGE = M32 ? 4096 : 2048;
};

// One work unit of the persistent schedule (a tile and a K-split of it);
// every field is wave-uniform.
struct Unit {
    int m0, n0;    // tile origin
    int split;     // K-split index
    int sbeg, nst; // first 128-K stage and number of stages of the split
    int valid;     // 0: past the end of this workgroup's unit list
    int e;         // expert (grouped GEMM; 0 otherwise)
    int rowlim;    // rows >= rowlim are not stored (the expert's or the matrix end)
};

// Chunk swizzle of an A pair slot: row r keeps its global 16-byte chunk c at
// physical chunk c ^ (r & 7).  A fragment read (16 rows, one chunk per row)
// then has no LDS bank conflicts on gfx950 (measured with SQ_LDS_BANK_CONFLICT:
// unswizzled 128-byte rows conflict 4-way, this pattern not at all).
__device__ __forceinline__ int a_swz(int r) { return r & 7; }

// Gap (after MFMA g of a stage's ng) at which VMEM item d of the stage's ni
// issues: the items are spread over gaps [rw + rw/2, ng - rw/2).
__host__ __device__ constexpr int item_gap(int d, int ni, int ng, int rw)
{
    const int span = ng - 2 * rw > 0 ? ng - 2 * rw : 1;
    const int gi = rw + rw / 2 + d * span / ni;
    return gi < ng ? gi : ng - 1;
}
// Items [first, ni) of a stage that issue in a later gap than item first-1.
// Loads that share a gap may be issued in either order (only the gaps are
// fenced), so only these are known to be issued after item first-1.
__host__ __device__ constexpr int items_after_gap_of(int first, int ni, int ng, int rw)
{
    int n = 0;
    for (int d = first; d < ni; ++d) n += item_gap(d, ni, ng, rw) > item_gap(first - 1, ni, ng, rw) ? 1 : 0;
    return n;
}

// Persistent B-direct kernel: gridDim.x workgroups (at most one resident
// set per CU) walk work units id = blockIdx.x + i*gridDim.x.  Per unit the
// K loop runs n_st4 = round_up(sps, 4) stages (stages past the split end are
// dead: their loads read zeros).  The software pipeline crosses unit
// boundaries: the last four stages of a unit already prefetch the next
// unit's first stages and scale group, so the next unit's MFMAs start right
// after this unit's epilogue, and no workgroup relaunch (with its pipeline
// fill and store drain) happens between tiles.
//
// Schedule of a stage ls (u = ls & 3): MFMAs of stage ls; loads of B stage
// ls+3 and (odd ls) scale group (ls+3)/2; the A DMA of half (ls & 1) of the
// pair starting at stage (ls & ~1) + 4.  A pair slot is rewritten only after
// the barrier that follows the last read of its previous pair, and the
// stage-top waits cover every pair before its first read, with three slots.
// The slot of a pair is its running index mod 3 across units: the three slot
// pointers rotate by one position per 4-stage iteration (two pairs).  Tiles
// with four slots (BdShape::NSLOT) swap them pairwise instead, and their even
// stages need no barrier.  A fragment and
// scale reads are explicit ds_read instructions with counted lgkmcnt waits
// (the compiler would otherwise make them wait for the A DMA into the
// dynamically chosen slot).
//
// GROUPED: the units are the tiles of every expert's row block (the tile
// grid of expert e is ceil(rows_e / BM) x tiles_n); B, its scales and the B
// factors are offset to expert e, and rows past the expert's end, which
// belong to the next expert, are computed but not stored.
//
// AFF: the bf16 epilogue applies MBS factors and alpha (1), and the column
// bias (2).  Each form is a separate instantiation so that the plain
// epilogue's register allocation is not sized for the scaled one's extra
// live values (which would spill into scratch, and each scratch reload
// waits on the next unit's outstanding DMAs); the form without a bias saves
// a third of the scaled epilogue's per-element arithmetic.
template <class T, bool GEN, bool SPLIT, bool GROUPED = false, int AFF = 0>
__global__ void __launch_bounds__(T::NT) gemm_bdirect_kernel(const GemmArgs p)
{
    static_assert(!(GROUPED && SPLIT), "grouped GEMM runs without K splits");
    static_assert(!(AFF && SPLIT), "split launches write fp32 partial sums");
    static_assert(AFF >= 0 && AFF <= 2, "epilogue form");
    static_assert(!T::M32 || (!GEN && !SPLIT), "M32 tiles: whole-K, single-split");
    __shared__ __attribute__((aligned(1024))) uint8_t pa0[T::PSLOT];
    __shared__ __attribute__((aligned(1024))) uint8_t pa1[T::PSLOT];
    __shared__ __attribute__((aligned(1024))) uint8_t pa2[T::PSLOT];
    __shared__ __attribute__((aligned(T::NSLOT == 4 ? 1024 : 4))) uint8_t pa3[T::NSLOT == 4 ? T::PSLOT : 4];
    // MBS factor bytes of a unit (A rows at [0,256), B columns at [256,512)),
    // double-buffered by unit parity, and the byte -> fp32 factor table.
    __shared__ __attribute__((aligned(16))) uint8_t fbytes[2][T::FBW];
    __shared__ __attribute__((aligned(16))) uint16_t fbias[2][T::NBB * 128];
    __shared__ __attribute__((aligned(16))) uint8_t fjunk[1024];  // target of filler DMAs
    // Scale groups, double-buffered by group parity.
    __shared__ __attribute__((aligned(1024))) uint8_t sc0[T::SBUF];
    __shared__ __attribute__((aligned(1024))) uint8_t sc1[T::SBUF];
    __shared__ float ftab[256];
    // Epilogue staging, per wave: 16 rows x 128 bytes (STAGE_EPI shapes).
    __shared__ __attribute__((aligned(16))) uint8_t estage[T::STAGE_EPI ? T::NW : 1][T::EPI_STAGE];
    __shared__ uint32_t ftail;   // A factor bytes of rows Mdw.. M-1 (at most 3)
    // AFF: the unit's factors as fp32, converted once per unit from fbytes
    // (columns: f(b); rows: f(a) * alpha), double-buffered by unit parity.
    __shared__ __attribute__((aligned(16))) float fcolf[AFF ? 2 : 1][AFF ? T::BN : 1];
    __shared__ __attribute__((aligned(16))) float frowf[AFF ? 2 : 1][AFF ? T::BM : 1];
    // Pair slots of the current 4-stage iteration: q0 (pair 0, stages 0-1),
    // q1 (pair 1, stages 2-3), q2 (pair 2, DMA'd by stages 0-1); pair 3 (DMA'd
    // by stages 2-3) reuses q0.  Next iteration: (q0, q1, q2) <- (q2, q0, q1).
    // Four slots: pair 3 goes to q3, and (q0, q1, q2, q3) <- (q2, q3, q0, q1).
    uint8_t* q0 = pa0;
    uint8_t* q1 = pa1;
    uint8_t* q2 = pa2;
    uint8_t* q3 = nullptr;
    if constexpr (T::NSLOT == 4) q3 = pa3;
    auto qp = [&](auto K) __attribute__((always_inline)) -> uint8_t* {
        constexpr int k = decltype(K)::value & 3;
        if constexpr (k == 3 && T::NSLOT == 4) return q3;
        else if constexpr (k == 0 || k == 3) return q0;
        else if constexpr (k == 1) return q1;
        else return q2;
    };

    PhaseClock ph;
    ph.start();
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = w / T::WGN, wn = w % T::WGN;

    const int K = p.K, Kp = K >> 1;
    const int S_total = (K + 127) >> 7;
    const int n_st4 = (p.sps + 3) & ~3;
    // Grouped: the first M-tile index of each expert (prefix sums), in LDS.
    __shared__ int gtile[GROUPED ? kMaxGroups + 1 : 1];
    __shared__ int gscan[GROUPED ? T::NT : 1];
    int tiles_m = p.tiles_m;
    // Expert e's rows, clamped into [0, M]: the offsets come from the device
    // and are not checked on the host, so no offset may move a store outside
    // the output or raise the tile count past E * ceil(M / BM).
    auto g_beg = [&](int e) __attribute__((always_inline)) { return min(max(p.groups[e], 0), p.M); };
    auto g_end = [&](int e) __attribute__((always_inline)) {
        return min(max(p.groups[e + 1], g_beg(e)), p.M);
    };
    // M-tiles of expert e.  An expert whose first row is not a multiple of 32
    // gets none (its rows are not written): the shuffled A scales come in
    // 32-row groups, and a tile starting inside one would read the wrong
    // scale bytes.  mbs_gemm_a4w4_check_groups reports such offsets.
    auto g_tiles = [&](int e) __attribute__((always_inline)) {
        const int b = g_beg(e);
        return (b & 31) ? 0 : (g_end(e) - b + T::BM - 1) / T::BM;
    };
    if constexpr (GROUPED) {
        // Prefix sums over the whole workgroup: thread t sums the experts of
        // its contiguous chunk, the chunk sums are scanned in LDS
        // (Hillis-Steele), and each thread writes its chunk's prefixes.
        const int E = p.n_groups;
        const int per = (E + T::NT - 1) / T::NT;
        const int e0 = min((int)threadIdx.x * per, E), e1 = min(e0 + per, E);
        int sum = 0;
        for (int e = e0; e < e1; ++e) sum += g_tiles(e);
        gscan[threadIdx.x] = sum;
        __syncthreads();
        for (int d = 1; d < T::NT; d <<= 1) {
            const int v = (int)threadIdx.x >= d ? gscan[threadIdx.x - d] : 0;
            __syncthreads();
            gscan[threadIdx.x] += v;
            __syncthreads();
        }
        int run = gscan[threadIdx.x] - sum;
        for (int e = e0; e < e1; ++e) {
            gtile[e] = run;
            run += g_tiles(e);
        }
        if (threadIdx.x == T::NT - 1) gtile[E] = gscan[T::NT - 1];
        __syncthreads();
        tiles_m = gtile[E];
    }
    const int tiles = tiles_m * p.tiles_n;
    const int units = tiles * p.splits;
    // A grouped launch whose experts are all empty (or skipped) has no work;
    // every workgroup leaves before its first load.
    if (units == 0) return;
    const int G = gridDim.x;
    // Workgroups are dispatched round-robin over the 8 XCDs (private L2s).
    // With G % 8 == 0 the ids of one XCD are those with id % 8 == x; map
    // them onto a contiguous range of units so that the units an XCD runs
    // concurrently form a compact block of tiles (GROUP tile-rows tall).
    // With at most one unit per workgroup (units <= G) each workgroup's only
    // unit is its own id, so the map also holds for any G (the units past
    // the last multiple of 8 keep their ids).
    const bool remap = (G & 7) == 0 || units <= G;
    const int units8 = units & ~7;
    auto unit_of = [&](int id) __attribute__((always_inline)) {
        Unit u;
        u.valid = id < units;
        int x = min(id, units - 1);
        if (remap && x < units8) x = (x & 7) * (units8 >> 3) + (x >> 3);
        u.split = x / tiles;
        const int t = x - u.split * tiles;
        // 4 tile-rows: the ~32 tiles an XCD runs at once are 4 rows x 8
        // columns.  Measured against 1, 2, 8, 16 and 32 rows (graph-replayed,
        // same bytes): 8192^3 ran 0.6-2% faster than with 8 and 4-5% faster
        // than with 1 or 32; the other model shapes moved within +-3%.
        constexpr int GROUP = 4;
        const int grp = t / (GROUP * p.tiles_n);
        const int first_m = grp * GROUP;
        const int gsz = min(tiles_m - first_m, GROUP);
        const int tin = t - grp * GROUP * p.tiles_n;
        const int gm = first_m + tin % gsz;   // M-tile index
        u.n0 = (tin / gsz) * T::BN;
        u.sbeg = u.split * p.sps;
        u.nst = min(p.sps, S_total - u.sbeg);
        if constexpr (GROUPED) {
            // the expert of M-tile gm: the last e with gtile[e] <= gm
            int lo = 0, hi = p.n_groups - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (gtile[mid] <= gm) lo = mid;
                else hi = mid - 1;
            }
            u.e = lo;
            u.m0 = g_beg(lo) + (gm - gtile[lo]) * T::BM;
            u.rowlim = g_end(lo);   // rows past it are not stored
        } else {
            u.e = 0;
            u.m0 = gm * T::BM;
            u.rowlim = p.M;
        }
        return u;
    };

    // Whole-operand resources; the unit's tile origin and the stage go into
    // the scalar offset, a dead stage uses soffset = kOOB (reads zeros).
    // The bounds keep every voffset + soffset below 2^32 (checked on the host).
    const int Mpad = (p.M + 31) & ~31, Npad = (p.N + 31) & ~31;
    const int nexp = GROUPED ? p.n_groups : 1;   // stacked B blocks
    const rsrc_t rA = make_rsrc(p.A, (uint32_t)(p.M * Kp));
    const rsrc_t rB = make_rsrc(p.B, (uint32_t)(nexp * p.N * Kp));
    const rsrc_t rAs = make_rsrc(p.As, (uint32_t)(Mpad * p.snp));
    const rsrc_t rBs = make_rsrc(p.Bs, (uint32_t)(nexp * Npad * p.snp));
    int sa[2][T::SA], sb[2][T::SB];  // scale dwords of two groups (set = group & 1)

    // Per-lane offsets within a tile, fixed for the whole kernel.
    // A DMA j of a pair half: lane i -> row 8j + i/8 of the half, physical
    // chunk i%8, which holds global chunk (i%8) ^ swz(row); swz(row) = i/8
    // since the half starts at a multiple of 8 rows (ADEAL: j counts the
    // DMAs of the whole pair, rows 8j + i/8 of the slot).
    // cA: the lane's K-byte offset in the pair (K-tail and dead-stage masks).
    uint32_t voA[T::NVA], cA[T::NVA];
    static_for<T::NVA>([&](auto d) {
        const int j = w * (T::ADEAL ? T::DAP : T::DA) + d;
        const int c = (lane & 7) ^ (lane >> 3);
        cA[d] = (uint32_t)(c * 16);
        voA[d] = (uint32_t)((8 * j + (lane >> 3)) * Kp + c * 16);
    });
    // A fragment read of half h: lane L -> row L%16 of the fragment, global
    // chunk 4h + L/16, at its swizzled position.  M32: of 64-K step k of the
    // pair: lane L -> row L%32, chunk 2k + L/32.
    uint32_t loA[T::M32 ? 4 : 2];
    if constexpr (T::M32) {
        static_for<4>([&](auto Kk) {
            constexpr int k = decltype(Kk)::value;
            loA[k] = (uint32_t)((lane & 31) * 128 + (((2 * k + (lane >> 5)) ^ a_swz(lane & 31)) * 16));
        });
    } else {
        static_for<2>([&](auto H) {
            constexpr int h = decltype(H)::value;
            loA[h] = (uint32_t)((lane & 15) * 128 + (((4 * h + (lane >> 4)) ^ a_swz(lane & 15)) * 16));
        });
    }
    // B: the wave's fragment j is 16 rows at n0 + wn*WN + 16j.  M32: fragment
    // j = s*FN32 + j32 is the 32 rows at n0 + wn*WN + 32*j32 for 64-K step s
    // of the stage; in the (16,16) preshuffle lane L's 16 bytes (row L%32, K
    // bytes 32s + 16*(L/32)..) sit at 16-row group (L%32)/16, 512-byte block
    // s, 256-byte half L/32, offset 16*(L%16).
    uint32_t voB[T::FN];
    static_for<T::FN>([&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (T::M32) {
            constexpr int s = j / T::FN32, j32 = j % T::FN32;
            voB[j] = (uint32_t)((wn * T::FN + 2 * j32 + ((lane >> 4) & 1)) * K * 8 + s * 512 +
                                (lane >> 5) * 256 + (lane & 15) * 16);
        } else {
            voB[j] = (uint32_t)((wn * T::FN + j) * K * 8 + lane * 16);
        }
    });
    // Scale DMA i of this wave is the workgroup's DMA k = w + NW*i: k < NSDA
    // gathers A chunks 4k..4k+3 (lane group lane/16 -> chunk), the next NSDB
    // gather B chunks, any further k is a filler.  Lanes past the last chunk
    // read out of range: 2^30 is above every scale buffer (M*K/2 < 2^31), and
    // plus any scalar offset used here (< 2^31 + 2^20) stays below 2^32.
    uint32_t voSD[T::NSDW];
    static_for<T::NSDW>([&](auto i) {
        const int k = w + T::NW * i;
        const int ch = 4 * (k < T::NSDA ? k : k - T::NSDA) + (lane >> 4);
        const bool ok = k < T::NSDA ? ch < T::CA : (k < T::NSD && ch < T::CB);
        voSD[i] = ok ? (uint32_t)(ch * 32 * p.snp + (lane & 15) * 16) : 0x40000000u;
    });
    auto sbuf = [&](auto B) __attribute__((always_inline)) -> uint8_t* {
        if constexpr ((decltype(B)::value & 1) == 0) return sc0;
        else return sc1;
    };
    // DMA i of a scale group (target t: its unit and group) into buffer BUF.
    // Whether this wave's DMA i gathers A or B chunks, or is a filler, is
    // fixed for the kernel: resource, destination and offset are selects,
    // not branches.
    auto scale_dma = [&](auto BUF, auto I, const auto& t) __attribute__((always_inline)) {
        constexpr int i = decltype(I)::value;
        const int k = w + T::NW * i;
        const bool real = (T::NSDW * T::NW == T::NSD) || k < T::NSD;
        const bool isa = k < T::NSDA;
        uint8_t* dst = real ? sbuf(BUF) + k * 1024 : fjunk;
        dma16s(isa ? rAs : rBs, dst, voSD[i], real ? (isa ? t.as : t.bs) : kOOB);
    };
    // LDS addresses of this wave's scale dwords in each scale buffer (dword
    // k of the A or B part at + k*256).  M32: lane L reads dwords
    // 16*(L/32) + L%16 and 32 + that of each 32-row chunk (see scale32).
    const int slane = T::M32 ? ((lane >> 5) * 16 + (lane & 15)) * 4 : lane * 4;
    const uint32_t scA[2] = {lds_addr(sc0) + (uint32_t)((((wm * T::WM) >> 5)) * 256 + slane),
                             lds_addr(sc1) + (uint32_t)((((wm * T::WM) >> 5)) * 256 + slane)};
    const uint32_t scB[2] = {
        lds_addr(sc0) + (uint32_t)(T::NSDA * 1024 + ((wn * T::WN) >> 5) * 256 + slane),
        lds_addr(sc1) + (uint32_t)(T::NSDA * 1024 + ((wn * T::WN) >> 5) * 256 + slane)};
    // M32 scales: the four 64-K steps of a 256-K group need, in lane L, the
    // E8M0 bytes of (row L%32, block 2k + L/32), k = 0..3.  In the shuffled
    // layout they are bytes t and t+2 (t = (L%32)/16) of the two dwords read
    // above; v_perm packs them so that byte k serves step k (op_sel = k).
    const uint32_t perm_sel = ((lane >> 4) & 1) ? 0x07030501u : 0x06020400u;
    auto scale32 = [&](int d0, int d1) __attribute__((always_inline)) {
        return (int)__builtin_amdgcn_perm((uint32_t)d1, (uint32_t)d0, perm_sel);
    };
    // GEN kernels also run shapes without a K tail (dead stages only).
    const bool ktail = (K & 127) != 0;
    const bool hi_lane = lane >= 32;
    const uint32_t hi_bit = hi_lane ? kOOB : 0u;

    i32x4 rb[4][T::FN];     // B register ring (stage % 4)
    i32x4 ra[4];            // A fragment ring (fragment sequence % 4)
    using AccT = std::conditional_t<T::M32, f32x16, f32x4>;
    AccT acc[T::AR][T::AC];
    static_for<T::AR>([&](auto i) {
        static_for<T::AC>([&](auto j) { acc[i][j] = AccT{}; });
    });
    // M32: packed scales of the two groups in flight (set = group & 1)
    int spa[2][T::M32 ? T::FM32 : 1], spb[2][T::M32 ? T::FN32 : 1];

    Unit cur = unit_of(blockIdx.x);
    Unit nxt = unit_of(blockIdx.x + G);
    // Operand offsets of a unit's first stage and its live stage count (0
    // past the end of the unit list), computed once per unit so that the
    // per-stage load targets are a few selects and adds (no branches).
    struct Orig {
        uint32_t a, b, as, bs;
        int nst, sbeg;
    };
    auto orig_of = [&](const Unit& un) __attribute__((always_inline)) {
        Orig o;
        o.a = un.valid ? (uint32_t)(un.m0 * Kp + un.sbeg * 64) : kOOB;
        o.b = un.valid ? (uint32_t)((un.e * p.N + un.n0) * Kp + un.sbeg * 1024) : kOOB;
        o.as = un.valid ? (uint32_t)(un.m0 * p.snp + (un.sbeg >> 1) * 256) : kOOB;  // sbeg is even
        o.bs = un.valid ? (uint32_t)((un.e * Npad + un.n0) * p.snp + (un.sbeg >> 1) * 256) : kOOB;
        o.nst = un.valid ? un.nst : 0;
        o.sbeg = un.sbeg;
        return o;
    };
    Orig ocur = orig_of(cur), onxt = orig_of(nxt);

    // Load target for local stage x of the current unit (x >= n_st4: stage
    // x - n_st4 of the next unit).
    struct Tgt {
        uint32_t a, b, as, bs;  // scalar offsets (kOOB when dead)
        uint32_t tv;            // per-lane K-tail bit (GEN only)
    };
    auto target = [&](int x) __attribute__((always_inline)) {
        const bool in_cur = x < n_st4;
        const int xl = in_cur ? x : x - n_st4;
        const Orig& o = in_cur ? ocur : onxt;
        const bool live = xl < o.nst;
        Tgt t;
        t.a = live ? o.a + (uint32_t)xl * 64u : kOOB;
        t.b = live ? o.b + (uint32_t)xl * 1024u : kOOB;
        t.as = live ? o.as + (uint32_t)(xl >> 1) * 256u : kOOB;
        t.bs = live ? o.bs + (uint32_t)(xl >> 1) * 256u : kOOB;
        t.tv = 0;
        if constexpr (GEN) {
            const int s = o.sbeg + xl;
            uint32_t v = ((uint32_t)(live & ktail & (s == S_total - 1)) << 31) & hi_bit;
            asm volatile("" : "+v"(v));
            t.tv = v;
        }
        return t;
    };
    // A DMA w*DA + d of half H of pair K (of the iteration) into its slot.  `soff`: the
    // pair's scalar offset (kOOB + small when dead); GEN kernels also mask
    // the lanes whose chunk lies past the pair's `vb` live bytes (K tail,
    // dead stage).  When AF is not a multiple of the wave count, the surplus
    // DMAs read out of range into fjunk, so every wave issues DA of them;
    // ADEAL tiles issue DMA w*DAP + d (stage H = 0) or w*DAP + DAE + d (H = 1)
    // of the whole pair instead.
    auto a_dma = [&](auto PK, auto H, auto D, uint32_t soff, int vb) __attribute__((always_inline)) {
        constexpr int d = decltype(D)::value, h = decltype(H)::value;
        if constexpr (T::ADEAL) {   // rows 8 jd .. of the slot, no fillers
            constexpr int dd = (h ? T::DAE : 0) + d;
            const int jd = w * T::DAP + dd;
            uint32_t vo = voA[dd];
            if constexpr (GEN) vo |= ((int)cA[dd] >= vb) ? kOOB : 0u;
            dma16s(rA, qp(PK) + jd * 1024, vo, soff);
        } else {
            const int j = w * T::DA + d;
            uint32_t vo = voA[d];
            if constexpr (GEN) vo |= ((int)cA[d] >= vb) ? kOOB : 0u;
            const uint32_t so = soff + (uint32_t)(h * (T::BM / 2) * Kp);
            if (T::AF % T::NW == 0 || j < T::AF)
                dma16s(rA, qp(PK) + h * (T::BM / 2) * 128 + j * 1024, vo, so);
            else
                dma16s(rA, fjunk, voA[d], kOOB);
        }
    };
    // Scalar offset and live bytes of the A pair DMA'd at local stage ls
    // (the pair starting at stage (ls & ~1) + 4, possibly the next unit's).
    struct TgtA {
        uint32_t a;
        int vb;
    };
    auto target_a = [&](int ls) __attribute__((always_inline)) {
        const int xp = (ls & ~1) + 4;
        const bool in_cur = xp < n_st4;
        const int xl = in_cur ? xp : xp - n_st4;
        const Orig& o = in_cur ? ocur : onxt;
        const int kend = min((o.sbeg + o.nst) * 64, Kp);   // live K bytes end (o.nst = 0: none)
        TgtA t;
        t.vb = kend - (o.sbeg + xl) * 64;
        t.a = t.vb > 0 ? o.a + (uint32_t)xl * 64u : kOOB;
        return t;
    };
    // VMEM items issued at local stage ls (static slot u = ls & 3), in this
    // order: DAE / DAO A-DMAs, on odd stages the NSDW scale DMAs of 256-K
    // group (ls+3)/2 into buffer ((ls+3)/2) & 1, then the FN B-loads for
    // stage ls+3 (last, so that odd stages can leave them in flight).
    auto issue_item = [&](auto U, auto D, const Tgt& t3, const TgtA& ta)
        __attribute__((always_inline)) {
        constexpr int u = decltype(U)::value;
        constexpr int d = decltype(D)::value;
        constexpr int DAu = (u & 1) ? T::DAO : T::DAE;
        constexpr int NSu = (u & 1) ? T::NSDW : 0;
        if constexpr (d < DAu) {
            a_dma(std::integral_constant<int, (u >> 1) + 2>{}, std::integral_constant<int, u & 1>{},
                  std::integral_constant<int, d>{}, ta.a, ta.vb);
        } else if constexpr (d < DAu + NSu) {
            scale_dma(std::integral_constant<int, ((u + 3) >> 1) & 1>{},
                      std::integral_constant<int, d - DAu>{}, t3);
        } else {
            constexpr int j = d - DAu - NSu;
            rb[(u + 3) & 3][j] = load16s(rB, voB[j] | t3.tv, t3.b);
        }
    };
    // Issues per stage: NI_EVEN on even stages, NI_ODD on odd ones.
    constexpr int NI_EVEN = T::DAE + T::FN;
    constexpr int NI_ODD = T::DAO + T::FN + T::NSDW;
    // B loads of an odd stage known to issue after its scale DMAs.
    constexpr int NB_LATE = items_after_gap_of(T::DAO + T::NSDW, NI_ODD, T::FM * T::RW, T::RW);
    // VMEM operations of an epilogue, all issued unconditionally: the bf16
    // stores (one per fragment pair and row block) and the factor DMAs of the
    // next unit (FD per wave).  vmcnt retires in issue order, so the first
    // wait after an epilogue can leave them in flight (SPLIT: its fp32
    // partial stores exceed the 6-bit count and are waited for).
    constexpr int FD = (T::NW == 1 ? 2 : 1) + T::FBB;   // factor + bias DMAs per wave
    constexpr int EPI_OPS = SPLIT ? 0 : T::FM * (T::FN / 2) + FD;
    static_assert(NI_EVEN + T::FN + EPI_OPS <= 63 && NI_EVEN + NI_ODD <= 63, "vmcnt is 6 bits");

    // A fragment x of the wave, half H of pair K of the iteration -> ra[R].
    // M32: fragment row x is 32-row block x % FM32 at 64-K step
    // 2H + x / FM32 of the pair.
    auto read_a = [&](auto PK, auto H, auto X, auto R) __attribute__((always_inline)) {
        constexpr int x = decltype(X)::value, h = decltype(H)::value;
        if constexpr (T::M32)
            ra[decltype(R)::value] = ds_read16<(x % T::FM32) * 4096>(lds_addr(qp(PK)) + loA[2 * h + x / T::FM32]);
        else
            ra[decltype(R)::value] =
                ds_read16<x * 2048>(lds_addr(qp(PK)) + loA[h] + (uint32_t)(wm * T::FM * 2048));
    };

    // One scale dword of the group in buffer BUF -> register set SET
    // (k < SA: A dword k, else B dword k - SA).
    auto read_scale = [&](auto BUF, auto SET, auto KI) __attribute__((always_inline)) {
        constexpr int set = decltype(SET)::value, k = decltype(KI)::value, b = decltype(BUF)::value & 1;
        constexpr int st = T::M32 ? 128 : 256;   // M32: two dwords 128 bytes apart per 32-row chunk
        if constexpr (k < T::SA) sa[set][k] = ds_read4<k * st>(scA[b]);
        else sb[set][k - T::SA] = ds_read4<(k - T::SA) * st>(scB[b]);
    };
    static_assert(T::FM >= 4, "the A look-ahead and scale-read schedule needs 4+ fragments");
    // Gap of scale read k of an odd stage: spread over [RW, (FM-2)*RW), so
    // every scale read is older than the two look-ahead fragment reads that
    // end the stage (which makes the wait of the next stage's first MFMA
    // cover them).  RW: MFMAs (= gaps) per fragment row.
    constexpr int NSR = T::SA + T::SB;
    constexpr int RW = T::RW;
    constexpr auto scale_gap = [](int k) constexpr { return RW + (k * ((T::FM - 3) * RW)) / NSR; };
    // Scale reads of an odd stage at gaps in [g0, g1).
    constexpr auto scales_in = [scale_gap](int g0, int g1) constexpr {
        int n = 0;
        for (int k = 0; k < NSR; ++k) n += (scale_gap(k) >= g0 && scale_gap(k) < g1) ? 1 : 0;
        return n;
    };

    // Load targets of the stage three ahead.  GEN kernels (dead stages or a
    // K tail possible) compute them per stage with target(); the others keep
    // them in `run` and advance it by constant steps, switching to the next
    // unit's origin when the load stage crosses the unit end.
    Tgt run{};
    TgtA runA{};

    // A stage issues its FM x FN MFMAs one by one; the gap after MFMA g gets
    // at most a few other instructions, spread so that with one wave per
    // SIMD the matrix pipe is never starved by a burst of issues:
    //   gap FN*c      the look-ahead A read (fragment c+2, possibly of the next stage)
    //   gap item_gap  the VMEM items (A DMAs, scale DMAs on odd stages, B loads)
    //   gap scale_gap the next scale group's dwords (odd stages)
    // FIRST: the unit's first stage; its MFMAs start the accumulators from 0.
    // `post`: stage of the first iteration of a unit that follows an
    // epilogue.  Its u = 0 wait and barrier were done before that epilogue;
    // its u = 1 wait also leaves the epilogue's EPI_OPS operations in flight.
    auto stage = [&](auto U, auto FIRST, int ls, bool post) __attribute__((always_inline)) {
        constexpr int u = decltype(U)::value;
        constexpr bool first = decltype(FIRST)::value;
        constexpr int h = u & 1, sset = (u >> 1) & 1;
        constexpr int NI = ((u & 1) == 0) ? NI_EVEN : NI_ODD;   // issues of this stage
        constexpr int NIP = ((u & 1) == 0) ? NI_ODD : NI_EVEN;  // issues of the previous one
        constexpr int NG = T::FM * RW;                          // MFMAs (= gaps) per stage
        // Stage-top wait.  Odd stages read the next scale group, DMA'd two
        // stages ago: everything issued two or more stages ago has landed
        // except that stage's B loads issued after its last scale DMA (B is
        // issued last on odd stages, and B of stage ls+1 is not needed yet).
        // Even stages need only their B (issued three stages ago) and A
        // halves DMA'd three or more stages ago: the two previous stages'
        // issues may still be in flight.
        constexpr int WAITN = (u & 1) ? NIP + NB_LATE : NI_ODD + NI_EVEN;
        // Four slots: the even stages' data (three stages old) was published
        // by the previous odd stage's barrier, and their DMAs rewrite a slot
        // last read before it: a per-wave wait (for B) suffices.
        constexpr bool BAR = (u & 1) || T::NSLOT == 3;
        ph.mark((u == 0 && post) ? kPhNext : kPhBody);
        ph.stage();
        if constexpr (u == 0) {
            if (!post) {
                wait_vmcnt<WAITN>();
                ph.mark(kPhWait);
                if constexpr (BAR) barrier();
                ph.mark(kPhBar);
            }
        } else if constexpr (u == 1) {
            if (post) wait_vmcnt<WAITN + EPI_OPS>();
            else wait_vmcnt<WAITN>();
            ph.mark(kPhWait);
            barrier();
            ph.mark(kPhBar);
        } else {
            wait_vmcnt<WAITN>();
            ph.mark(kPhWait);
            if constexpr (BAR) barrier();
            ph.mark(kPhBar);
        }
        __builtin_amdgcn_sched_barrier(0);
        Tgt t3;
        TgtA ta;
        if constexpr (GEN) {
            t3 = target(ls + 3);
            ta = target_a(ls);
        } else {
            if constexpr (u == 1) {  // the only stage whose B stage can be a unit's first
                const bool sw = ls + 3 == n_st4;
                run.b = sw ? onxt.b : run.b;
                run.as = sw ? onxt.as : run.as;
                run.bs = sw ? onxt.bs : run.bs;
            }
            if constexpr (u == 0) {  // the only stage whose A pair can be a unit's first
                runA.a = ls + 4 == n_st4 ? onxt.a : runA.a;
            }
            t3 = run;
            ta = runA;
        }
        int sav[T::SA], sbv[T::SB];
        static_for<T::SA>([&](auto i) { sav[i] = sa[sset][i]; });
        static_for<T::SB>([&](auto j) { sbv[j] = sb[sset][j]; });
        if constexpr (GEN) {
            // The selects read the scale registers: wait for their ds_reads
            // first (only fragment 1's read, the youngest, may stay pending).
            constexpr int ar0 = (T::FM * u) & 3;
            wait_lgkm_for<1>(ra[ar0]);
            static_for<T::SA>([&](auto i) { tie_after(sav[i]); });
            static_for<T::SB>([&](auto i) { tie_after(sbv[i]); });
            const bool tail = ktail && ls < cur.nst && cur.sbeg + ls == S_total - 1 && hi_lane;
            static_for<T::SA>([&](auto i) { sav[i] = tail ? 0x7F7F7F7F : sav[i]; });
            static_for<T::SB>([&](auto j) { sbv[j] = tail ? 0x7F7F7F7F : sbv[j]; });
        }

        static_for<NG>([&](auto G_) {
            constexpr int g = decltype(G_)::value;
            // MFMA g multiplies A fragment c by B fragment j; k is its place
            // in the fragment row.  Odd rows walk the B fragments backwards,
            // so consecutive MFMAs always share an operand (at a row change
            // the B fragment stays): fewer operand changes on the matrix
            // pipe's inputs, whose switching activity sets the power-limited
            // clock under sustained load.
            constexpr int c = g / RW, k = g % RW;
            constexpr int j = (c & 1) ? RW - 1 - k : k;
            constexpr int ar = (T::FM * u + c) & 3;
            using PKu = std::integral_constant<int, (u >> 1)>;        // pair of this stage
            using PKn = std::integral_constant<int, ((u + 1) >> 1)>;  // pair of the next
            // Fragment c was read at gap (c-2)*FN (of the previous stage for
            // c < 2).  LDS reads younger than it: the next fragment read and
            // (odd stages) the scale reads since that gap; the first MFMA of
            // the chunk waits for the rest.  At c = 0 that also covers the
            // scales the stage uses (read before the look-ahead reads).
            constexpr int nyoung =
                1 + ((u & 1) && c >= 2 ? scales_in((c - 2) * RW, c * RW) : 0);
            constexpr int opb = (j & 1) + 2 * h;
            constexpr int opa = (c & 1) + 2 * h;
            if constexpr (T::M32) {
                // row c = (64-K step s of the stage, 32-row block c32); B
                // fragment jb = (s, 32-column block j); scale byte = the step
                // within the 256-K group.  The unit's first stage starts each
                // accumulator at s = 0.
                constexpr int s = c / T::FM32, c32 = c % T::FM32;
                constexpr int kst = 2 * h + s;
                constexpr int jb = s * T::FN32 + j;
                constexpr bool fresh = first && s == 0;
                const int pb = spb[sset][j], pa = spa[sset][c32];
                if constexpr (k == 0) {
                    if constexpr (fresh)
                        mfma32_fp4_first_w<kst, kst, nyoung>(acc[c32][j], rb[u][jb], ra[ar], pb, pa);
                    else
                        mfma32_fp4_w<kst, kst, nyoung>(acc[c32][j], rb[u][jb], ra[ar], pb, pa);
                } else {
                    if constexpr (fresh)
                        mfma32_fp4_first<kst, kst>(acc[c32][j], rb[u][jb], ra[ar], pb, pa);
                    else
                        mfma32_fp4<kst, kst>(acc[c32][j], rb[u][jb], ra[ar], pb, pa);
                }
            }
            // K-tail stages select scales with VALU ops: keep the wait states there.
            else if constexpr (k == 0) {
                if constexpr (first && !GEN)
                    mfma_fp4_first_w<opb, opa, nyoung>(acc[c][j], rb[u][j], ra[ar], sbv[j / 2], sav[c / 2]);
                else
                    mfma_fp4_w<opb, opa, nyoung, GEN>(acc[c][j], rb[u][j], ra[ar], sbv[j / 2], sav[c / 2]);
            } else {
                if constexpr (first && !GEN)
                    mfma_fp4_first<opb, opa>(acc[c][j], rb[u][j], ra[ar], sbv[j / 2], sav[c / 2]);
                else
                    mfma_fp4<opb, opa, GEN>(acc[c][j], rb[u][j], ra[ar], sbv[j / 2], sav[c / 2]);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (k == 0) {
                // look-ahead A read: fragment c+2 of this stage or of the next
                constexpr int xn = c + 2;
                if constexpr (xn < T::FM)
                    read_a(PKu{}, std::integral_constant<int, u & 1>{},
                           std::integral_constant<int, xn>{},
                           std::integral_constant<int, (T::FM * u + xn) & 3>{});
                else
                    read_a(PKn{}, std::integral_constant<int, (u + 1) & 1>{},
                           std::integral_constant<int, xn - T::FM>{},
                           std::integral_constant<int, (T::FM * u + xn) & 3>{});
            }
            // VMEM items over gaps [RW + RW/2, NG - RW/2)
            static_for<NI>([&](auto D) {
                if constexpr (item_gap(decltype(D)::value, NI, NG, RW) == g) issue_item(U, D, t3, ta);
            });
            // Odd stages: the next group's scale dwords (DMA'd two stages
            // ago), after this gap's fragment read.
            if constexpr ((u & 1) == 1) {
                static_for<NSR>([&](auto KI) {
                    if constexpr (scale_gap(decltype(KI)::value) == g)
                        read_scale(std::integral_constant<int, ((u + 1) >> 1) & 1>{},
                                   std::integral_constant<int, ((u + 1) >> 1) & 1>{}, KI);
                });
                // M32, last gap: pack the next group's scale bytes (their
                // dwords have landed; only the two look-ahead fragment reads
                // may still be pending), then the two wait states a VALU
                // write needs before an MFMA reads it.
                if constexpr (T::M32 && g == NG - 1) {
                    constexpr int ns = ((u + 1) >> 1) & 1;
                    wait_lgkm_for<2>(sa[ns][0]);
                    static_for<T::SA>([&](auto i) { tie_after(sa[ns][decltype(i)::value]); });
                    static_for<T::SB>([&](auto i) { tie_after(sb[ns][decltype(i)::value]); });
                    static_for<T::FM32>([&](auto i) {
                        constexpr int x = decltype(i)::value;
                        spa[ns][x] = scale32(sa[ns][2 * x], sa[ns][2 * x + 1]);
                    });
                    static_for<T::FN32>([&](auto J) {
                        constexpr int x = decltype(J)::value;
                        spb[ns][x] = scale32(sb[ns][2 * x], sb[ns][2 * x + 1]);
                    });
                    static_for<T::FM32>([&](auto i) { tie_after(spa[ns][decltype(i)::value]); });
                    static_for<T::FN32>([&](auto J) { tie_after(spb[ns][decltype(J)::value]); });
                    asm volatile("s_nop 1");
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        if constexpr (!GEN) {  // advance the running targets to stage ls+4
            run.b += 1024u;
            if constexpr ((u & 1) == 0) {  // load stage ls+3 was odd: next 256-K group
                run.as += 256u;
                run.bs += 256u;
            } else {                       // both halves of the A pair issued
                runA.a += 128u;
            }
        }
    };

    // MBS factors: bytes of a unit's rows and columns go to fbytes[par] by
    // LDS DMA (wave 0: A, the last wave: B; a single wave does both).  Every
    // wave issues exactly FD DMAs, the others (and every DMA without factors
    // or past the last unit) read out of range into fjunk, so the count is
    // the same for all waves and units.  The A range is cut to whole dwords;
    // the bytes of the at most 3 rows past it are read once, into ftail.
    const bool has_f = (p.Af != nullptr) && (p.Bf != nullptr);
    const int Mdw = p.M & ~3;
    const rsrc_t rAf = make_rsrc(p.Af, has_f ? (uint32_t)Mdw : 0u);
    const rsrc_t rBf = make_rsrc(p.Bf, has_f ? (uint32_t)(nexp * p.N) : 0u);
    // Wave 0 loads the A bytes, wave NW-1-c the B chunk c (columns 256c..),
    // every other wave a filler.
    auto factor_dma = [&](const Unit& un, int par) __attribute__((always_inline)) {
        const bool go = has_f && un.valid;
        if constexpr (T::NW == 1) {
            dma4s(rAf, &fbytes[par][0], (uint32_t)(un.m0 + lane * 4), go ? 0u : kOOB);
            dma4s(rBf, &fbytes[par][256], (uint32_t)(un.e * p.N + un.n0 + lane * 4), go ? 0u : kOOB);
        } else {
            const bool wa = w == 0;
            const int c = T::NW - 1 - w;            // B chunk of this wave
            const bool wb = !wa && c < T::NBC;
            uint8_t* dst = wa ? &fbytes[par][0] : (wb ? &fbytes[par][256 * (1 + c)] : fjunk);
            const rsrc_t r = wa ? rAf : rBf;
            const uint32_t off = (uint32_t)((wa ? un.m0 : un.e * p.N + un.n0 + 256 * c) + lane * 4);
            dma4s(r, dst, off, go && (wa || wb) ? 0u : kOOB);
        }
    };
    // Epilogue bias of a unit's columns -> fbias[par] (FBB DMAs per wave,
    // fillers into fjunk when there is no bias or no unit).
    const bool has_bias = p.bias != nullptr;
    if constexpr (AFF) {
        // The scaled epilogue reads its operands without branches: factor
        // 1.0 for every byte without factors, a bias of -0.0 (x + -0.0 == x,
        // signed zeros included) without a bias.  These writes are ordered
        // before the first epilogue by the prologue's barrier.
        for (int b = threadIdx.x; b < 256; b += T::NT) ftab[b] = has_f ? factor_of((uint32_t)b) : 1.0f;
        if (threadIdx.x == 0) {
            uint32_t t = 0;
            if (has_f) {
                const rsrc_t rAt = make_rsrc(p.Af, (uint32_t)p.M);
                for (int k = 0; k < p.M - Mdw; ++k) t |= (load1(rAt, (uint32_t)(Mdw + k)) & 255u) << (8 * k);
            }
            ftail = t;
        }
        if (!has_bias) {
            uint32_t* fb = reinterpret_cast<uint32_t*>(&fbias[0][0]);
            for (int k = threadIdx.x; k < T::NBB * 128; k += T::NT) fb[k] = 0x80008000u;
        }
    }
    const rsrc_t rBias = make_rsrc(p.bias, has_bias ? (uint32_t)(nexp * p.N * 2) : 0u);
    auto bias_dma = [&](const Unit& un, int par) __attribute__((always_inline)) {
        static_for<T::FBB>([&](auto I) {
            const int k = w + T::NW * decltype(I)::value;   // 128-column chunk
            const bool go = has_bias && un.valid && k < T::NBB;
            dma4s(rBias, go ? (uint8_t*)&fbias[par][k * 128] : fjunk,
                  (uint32_t)((un.e * p.N + un.n0 + k * 128) * 2 + lane * 4), go ? 0u : kOOB);
        });
    };
    // AFF: factor bytes of the unit in fbytes[par] -> fp32 (one table lookup
    // per row and column per unit, instead of one per element group in the
    // epilogue, where the data-dependent table reads collide in LDS banks).
    // Called by every thread once its unit's factor DMA is known to have
    // landed for all waves; the epilogue reads the results after the barriers
    // that follow.
    auto convert_factors = [&](int par_, int m0_) __attribute__((always_inline)) {
        if constexpr (AFF) {
            for (int c = threadIdx.x; c < T::BN; c += T::NT) fcolf[par_][c] = ftab[fbytes[par_][256 + c]];
            const uint32_t tail = ftail;
            for (int r = threadIdx.x; r < T::BM; r += T::NT) {
                const int gr = m0_ + r;
                const uint32_t b = gr >= Mdw ? (tail >> (8 * ((gr - Mdw) & 3))) & 255u : fbytes[par_][r];
                frowf[par_][r] = ftab[b] * p.alpha;
            }
        }
    };
    factor_dma(cur, 0);
    bias_dma(cur, 0);

    // ---- prologue: scale groups 0 and 1, A pair 0, B stage 0, A pair 1,
    // B stages 1 and 2 of the first unit (pair p is what local stage 2p-4
    // would DMA: target_a(2p - 4)).
    static_for<2>([&](auto P) {
        const Tgt t = target(2 * decltype(P)::value);
        static_for<T::NSDW>([&](auto i) { scale_dma(P, i, t); });
    });
    auto b_stage = [&](auto S) __attribute__((always_inline)) {
        constexpr int ps = decltype(S)::value;
        const Tgt tb = target(ps);
        static_for<T::FN>([&](auto j) { rb[ps][j] = load16s(rB, voB[j] | tb.tv, tb.b); });
    };
    auto a_pair = [&](auto P) __attribute__((always_inline)) {
        const TgtA t = target_a(2 * decltype(P)::value - 4);
        static_for<2>([&](auto H) {
            static_for<decltype(H)::value ? T::DAO : T::DAE>([&](auto d) { a_dma(P, H, d, t.a, t.vb); });
        });
    };
    a_pair(std::integral_constant<int, 0>{});
    b_stage(std::integral_constant<int, 0>{});
    a_pair(std::integral_constant<int, 1>{});
    b_stage(std::integral_constant<int, 1>{});
    b_stage(std::integral_constant<int, 2>{});
    // The first stage is entered as if stages "-2" and "-1" had run: wait
    // for everything but A pair 1 and B stages 1 and 2, then read the scales
    // of group 0 and A fragments 0 and 1.
    wait_vmcnt<T::DAE + T::DAO + 2 * T::FN>();
    barrier();
    static_for<NSR>([&](auto KI) {
        read_scale(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, KI);
    });
    read_a(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{},
           std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    read_a(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{},
           std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
    if constexpr (T::M32) {   // pack group 0's scale bytes (as the odd stages do for later groups)
        wait_lgkm_for<2>(sa[0][0]);
        static_for<T::SA>([&](auto i) { tie_after(sa[0][decltype(i)::value]); });
        static_for<T::SB>([&](auto i) { tie_after(sb[0][decltype(i)::value]); });
        static_for<T::FM32>([&](auto i) {
            constexpr int x = decltype(i)::value;
            spa[0][x] = scale32(sa[0][2 * x], sa[0][2 * x + 1]);
        });
        static_for<T::FN32>([&](auto J) {
            constexpr int x = decltype(J)::value;
            spb[0][x] = scale32(sb[0][2 * x], sb[0][2 * x + 1]);
        });
        static_for<T::FM32>([&](auto i) { tie_after(spa[0][decltype(i)::value]); });
        static_for<T::FN32>([&](auto J) { tie_after(spb[0][decltype(J)::value]); });
        asm volatile("s_nop 1");
    }
    if constexpr (!GEN) {
        run = target(3);
        runA = target_a(0);
    }

    const int row_l = wm * T::WM + (lane & 15);
    const int q = lane >> 4;
    int par = 0;
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using FT = std::integral_constant<bool, true>;
    using FF = std::integral_constant<bool, false>;
    auto rotate = [&]() __attribute__((always_inline)) {
        if constexpr (T::NSLOT == 4) {
            uint8_t* t = q0;
            q0 = q2;
            q2 = t;
            t = q1;
            q1 = q3;
            q3 = t;
            return;
        }
        uint8_t* t = q2;
        q2 = q1;
        q1 = q0;
        q0 = t;
    };
    ph.mark(kPhPro);
    for (int id = blockIdx.x; id < units; id += G) {
        {   // first iteration, peeled: its stage 0 starts the accumulators
            const bool post = id != (int)blockIdx.x;
            if constexpr (GEN) {  // K-tail kernels keep plain MFMAs: zero first
                static_for<T::FM>([&](auto i) {
                    static_for<T::FN>([&](auto j) { acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f}; });
                });
            }
            stage(I0{}, FT{}, 0, post);
            stage(I1{}, FF{}, 1, post);
            stage(I2{}, FF{}, 2, false);
            // the wait and barrier of stage 2 (four slots: 3) cover the
            // factor DMAs issued with the previous epilogue (stage 1's may
            // leave them in flight)
            if constexpr (T::NSLOT == 3) convert_factors(par, cur.m0);
            stage(I3{}, FF{}, 3, false);
            if constexpr (T::NSLOT == 4) convert_factors(par, cur.m0);
            rotate();
        }
        for (int ls0 = 4; ls0 < n_st4; ls0 += 4) {
            stage(I0{}, FF{}, ls0, false);
            stage(I1{}, FF{}, ls0 + 1, false);
            stage(I2{}, FF{}, ls0 + 2, false);
            stage(I3{}, FF{}, ls0 + 3, false);
            rotate();
        }
        // The next unit's first stage would wait and sync here; doing it now
        // also makes this unit's factor bytes (and the table) visible.
        ph.mark(kPhBody);
        ph.unit();
        wait_vmcnt<NI_ODD + NI_EVEN>();
        ph.mark(kPhWait);
        barrier();
        ph.mark(kPhBar);
        mfma_drain();
        static_for<T::AR>([&](auto i) {
            static_for<T::AC>([&](auto j) { pin_after_drain(acc[i][j]); });
        });

        // ---- epilogue of unit `cur` -------------------------------------
        // (read back as scalars: the store descriptors must be uniform, or
        // every store becomes a readfirstlane loop)
        const int m0u = __builtin_amdgcn_readfirstlane(cur.m0);
        const int rows_a = __builtin_amdgcn_readfirstlane(max(0, min(T::BM, cur.rowlim - cur.m0)));
        const int col_w = cur.n0 + wn * T::WN;
        if constexpr (SPLIT) {
            const rsrc_t rW = make_rsrc(p.ws + ((size_t)cur.split * p.M + m0u) * p.N,
                                        (uint32_t)(rows_a * p.N * 4));
            static_for<T::FN>([&](auto j) {
                const int c = col_w + j * 16;
                if (c < p.N) {
                    static_for<T::FM>([&](auto i) {
                        store16(rW, (uint32_t)(((row_l + i * 16) * p.N + c + q * 4) * 4), acc[i][j]);
                    });
                }
            });
        } else {
            const rsrc_t rO = make_rsrc(p.out + (size_t)m0u * p.N, (uint32_t)(rows_a * p.N * 2));
            // HF: scaled and shifted, out = C * (alpha * f(a_m) * f(b_n)) +
            // bias[n], with the table and bias set up for the cases without
            // factors or bias.  Otherwise the accumulators are converted as
            // they are.
            // (each form is defined only where it is used: their accumulator
            // expressions do not depend on the lambdas' own parameters)
            if constexpr (!T::M32) {
            auto epi = [&](auto HF, auto BZ) __attribute__((always_inline)) {
                constexpr bool hf = decltype(HF)::value;
                constexpr bool bz = hf && decltype(BZ)::value;   // a bias to add
                float fa[T::FM];
                if constexpr (hf) {
                    static_for<T::FM>([&](auto i) { fa[i] = frowf[par][row_l + i * 16]; });
                }
                // Fragment pair (j, j+1) covers 32 columns.  Lane (m, q) holds
                // columns 4q..4q+3 of each; after two rounds of lane swaps it
                // holds 8 consecutive columns 8q..8q+7 of the pair (16 bytes)
                // of row m.  PairEpi: the pair's factor and bias operands.
                struct PairEpi {
                    float f0[4], f1[4], z0[4], z1[4];
                };
                auto pair_setup = [&](auto J0) __attribute__((always_inline)) {
                    constexpr int j0 = decltype(J0)::value;
                    PairEpi e;
                    if constexpr (hf) {
                        const int cl = wn * T::WN + j0 * 16 + q * 4;   // lane's first column in the tile
                        const f32x4 c0 = *reinterpret_cast<const f32x4*>(&fcolf[par][cl]);
                        const f32x4 c1 = *reinterpret_cast<const f32x4*>(&fcolf[par][cl + 16]);
                        static_for<4>([&](auto K4) {
                            constexpr int k = decltype(K4)::value;
                            e.f0[k] = c0[k];
                            e.f1[k] = c1[k];
                        });
                    }
                    if constexpr (bz) {
                        const int cl = wn * T::WN + j0 * 16 + q * 4;
                        const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&fbias[par][cl]);
                        const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&fbias[par][cl + 16]);
                        const uint32_t u0 = w0[0], u1 = w0[1], u2 = w1[0], u3 = w1[1];
                        e.z0[0] = bf16_lo(u0); e.z0[1] = bf16_hi(u0); e.z0[2] = bf16_lo(u1); e.z0[3] = bf16_hi(u1);
                        e.z1[0] = bf16_lo(u2); e.z1[1] = bf16_hi(u2); e.z1[2] = bf16_lo(u3); e.z1[3] = bf16_hi(u3);
                    }
                    return e;
                };
                // bf16 bits of pair (j0, j0+1) of row fragment i, lane (m, q):
                // row m, columns 8q..8q+7 of the pair.
                auto pair_bits = [&](auto I, auto J0, const PairEpi& e, uint32_t (&o)[4])
                    __attribute__((always_inline)) {
                    constexpr int i = decltype(I)::value, j0 = decltype(J0)::value;
                    f32x4 v0 = acc[i][j0], v1 = acc[i][j0 + 1];
                    if constexpr (bz) {
                        static_for<4>([&](auto K4) {
                            constexpr int k = decltype(K4)::value;
                            v0[k] = add_nc(v0[k] * (fa[i] * e.f0[k]), e.z0[k]);
                            v1[k] = add_nc(v1[k] * (fa[i] * e.f1[k]), e.z1[k]);
                        });
                    } else if constexpr (hf) {
                        static_for<4>([&](auto K4) {
                            constexpr int k = decltype(K4)::value;
                            v0[k] = v0[k] * (fa[i] * e.f0[k]);
                            v1[k] = v1[k] * (fa[i] * e.f1[k]);
                        });
                    }
                    uint32_t x0 = pack_bf16x2(v0[0], v0[1]), x1 = pack_bf16x2(v0[2], v0[3]);
                    uint32_t y0 = pack_bf16x2(v1[0], v1[1]), y1 = pack_bf16x2(v1[2], v1[3]);
                    // round A: upper half of x <-> lower half of y
                    auto a0 = __builtin_amdgcn_permlane32_swap(x0, y0, false, false);
                    auto a1 = __builtin_amdgcn_permlane32_swap(x1, y1, false, false);
                    // round B: odd rows of x <-> even rows of y
                    auto b0s = __builtin_amdgcn_permlane16_swap(a0[0], a0[1], false, false);
                    auto b1s = __builtin_amdgcn_permlane16_swap(a1[0], a1[1], false, false);
                    o[0] = b0s[0]; o[1] = b1s[0]; o[2] = b0s[1]; o[3] = b1s[1];
                };
                auto vec_of = [](const uint32_t (&o)[4]) __attribute__((always_inline)) {
                    i32x4 v = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
                    return __builtin_bit_cast(f32x4, v);
                };
                // Stores go through a per-wave LDS staging area so that
                // consecutive lanes write consecutive 16-byte chunks of one
                // row.  In the swapped-operand MFMA layout lane (m, q) holds row
                // m, so a direct store has neighbouring lanes in 16 different
                // rows; staged, 8 neighbouring lanes cover one 128-byte line.
                // Measured (graph replays, same bytes): 0.95-0.99x the time of
                // the direct 16-row x 64-byte stores on 256x256 tiles, epilogue
                // 8.6K -> 6.8K cycles per tile at 8192^3.  Chunks are
                // XOR-swizzled by row (conflict-free writes and reads).  Stores
                // are issued unconditionally (EPI_OPS): a lane past N stores at
                // kOOB, which the hardware drops.  A wave's LDS accesses run in
                // order, so its next block may overwrite the area right after
                // the reads; the compiler's lgkmcnt wait before each store
                // covers the reads.
                uint8_t* const stg = estage[T::STAGE_EPI ? w : 0];
                if constexpr (!T::STAGE_EPI) {
                    // straight from registers: 16 rows x 64 bytes per store
                    static_for<T::FN / 2>([&](auto P2) {
                        constexpr int j0 = 2 * decltype(P2)::value;
                        const PairEpi e = pair_setup(std::integral_constant<int, j0>{});
                        const int c = col_w + j0 * 16;
                        // N % 16 == 0: the pair is all in, only its first half, or out
                        const bool store_ok = c < p.N && (c + 16 < p.N || q < 2);
                        static_for<T::FM>([&](auto I) {
                            constexpr int i = decltype(I)::value;
                            uint32_t u[4];
                            pair_bits(I, std::integral_constant<int, j0>{}, e, u);
                            const uint32_t o = (uint32_t)(((row_l + i * 16) * p.N + c + q * 8) * 2);
                            store16(rO, store_ok ? o : kOOB, vec_of(u));
                            __builtin_amdgcn_sched_barrier(0);
                        });
                    });
                    return;
                }
                // Fragment quads (j0..j0+3, 64 columns = one 128-byte line of a
                // row): lane (m, q) writes row m, chunks q (pair j0) and 4+q
                // (pair j0+2) of a 16 x 128-byte block; lane L reads back row
                // L/8 (+8 for the second store), chunk L%8.
                constexpr int NQ = T::FN / 4;
                static_for<NQ>([&](auto Q4) {
                    constexpr int j0 = 4 * decltype(Q4)::value;
                    const PairEpi e0 = pair_setup(std::integral_constant<int, j0>{});
                    const PairEpi e1 = pair_setup(std::integral_constant<int, j0 + 2>{});
                    const int m = lane & 15, r = lane >> 3, cc = lane & 7;
                    uint8_t* const w0 = stg + m * 128 + ((q ^ (m & 7)) * 16);
                    uint8_t* const w1 = stg + m * 128 + (((4 + q) ^ (m & 7)) * 16);
                    const uint8_t* const r0 = stg + r * 128 + ((cc ^ r) * 16);
                    const int col = col_w + j0 * 16 + cc * 8;   // N % 16 == 0
                    const bool store_ok = col < p.N;
                    // Software-pipelined by one block: block i+1 is converted
                    // while block i's staging round trip is in flight.
                    uint32_t u[4], v[4];
                    pair_bits(I0{}, std::integral_constant<int, j0>{}, e0, u);
                    pair_bits(I0{}, std::integral_constant<int, j0 + 2>{}, e1, v);
                    static_for<T::FM>([&](auto I) {
                        constexpr int i = decltype(I)::value;
                        *reinterpret_cast<f32x4*>(w0) = vec_of(u);
                        *reinterpret_cast<f32x4*>(w1) = vec_of(v);
                        const f32x4 x0 = *reinterpret_cast<const f32x4*>(r0);
                        const f32x4 x1 = *reinterpret_cast<const f32x4*>(r0 + 1024);
                        if constexpr (i + 1 < T::FM) {
                            pair_bits(std::integral_constant<int, i + 1>{}, std::integral_constant<int, j0>{}, e0, u);
                            pair_bits(std::integral_constant<int, i + 1>{}, std::integral_constant<int, j0 + 2>{}, e1, v);
                        }
                        const uint32_t o = (uint32_t)(((wm * T::WM + i * 16 + r) * p.N + col) * 2);
                        store16(rO, store_ok ? o : kOOB, x0);
                        store16(rO, store_ok ? o + (uint32_t)(8 * p.N * 2) : kOOB, x1);
                        // keep the accumulator reads of later blocks from being
                        // hoisted here (register pressure)
                        __builtin_amdgcn_sched_barrier(0);
                    });
                });
                // A trailing pair (FN % 4 == 2): a 16 x 64-byte block, lane L
                // reads back row L/4, chunk L%4 (4 neighbouring lanes per row).
                if constexpr (T::FN % 4 == 2) {
                    constexpr int j0 = T::FN - 2;
                    const PairEpi e = pair_setup(std::integral_constant<int, j0>{});
                    const int m = lane & 15, r = lane >> 2, cc = lane & 3;
                    uint8_t* const w0 = stg + m * 64 + ((q ^ ((m >> 1) & 3)) * 16);
                    const uint8_t* const r0 = stg + r * 64 + ((cc ^ ((r >> 1) & 3)) * 16);
                    const int col = col_w + j0 * 16 + cc * 8;
                    const bool store_ok = col < p.N;
                    static_for<T::FM>([&](auto I) {
                        constexpr int i = decltype(I)::value;
                        uint32_t u[4];
                        pair_bits(I, std::integral_constant<int, j0>{}, e, u);
                        *reinterpret_cast<f32x4*>(w0) = vec_of(u);
                        const f32x4 x0 = *reinterpret_cast<const f32x4*>(r0);
                        const uint32_t o = (uint32_t)(((wm * T::WM + i * 16 + r) * p.N + col) * 2);
                        store16(rO, store_ok ? o : kOOB, x0);
                        __builtin_amdgcn_sched_barrier(0);
                    });
                }
            };
            epi(std::integral_constant<bool, AFF != 0>{}, std::integral_constant<bool, AFF == 2>{});
            } else {
            // M32: acc[c32][j] of lane L holds row c32*32 + L%32 of the wave
            // tile, columns 32j + 8q + 4v + i (q = r/4, i = r%4, v = L/32).
            // One round of lane swaps (lane L <-> L+32) gives each lane 8
            // consecutive columns (16 bytes) of its row per column pair q,
            // q+1.  Each pair of 32-column blocks (a 128-byte line of 32
            // rows) goes through the wave's staging area, chunks XOR-swizzled
            // by row, and is stored with 8 neighbouring lanes per row: 4
            // stores per 32 rows.  A trailing single block (96-column wave
            // tiles) is staged as 32 x 64 bytes and stored with 4 lanes per
            // row: 2 stores.  Together FM * (FN / 2) stores (EPI_OPS).
            auto epi32 = [&](auto HF, auto BZ) __attribute__((always_inline)) {
                constexpr bool hf = decltype(HF)::value;
                constexpr bool bz = hf && decltype(BZ)::value;   // a bias to add
                constexpr int NL = T::FN32 / 2;   // whole 128-byte lines
                const int m = lane & 31, v = lane >> 5;
                uint8_t* const stg = estage[w];
                // the lane's column factors and bias words, read once for all
                // row blocks: columns 32j + 8q + 4v .. +3
                f32x4 fcol[hf ? T::FN32 : 1][hf ? 4 : 1];
                uint32_t zw[bz ? T::FN32 : 1][bz ? 4 : 1][2];
                if constexpr (hf) {
                    static_for<T::FN32>([&](auto J) {
                        static_for<4>([&](auto Q) {
                            constexpr int j = decltype(J)::value, q = decltype(Q)::value;
                            const int cl = wn * T::WN + 32 * j + 8 * q + 4 * v;
                            fcol[j][q] = *reinterpret_cast<const f32x4*>(&fcolf[par][cl]);
                            if constexpr (bz) {
                                const uint32_t* bw = reinterpret_cast<const uint32_t*>(&fbias[par][cl]);
                                zw[j][q][0] = bw[0];
                                zw[j][q][1] = bw[1];
                            }
                        });
                    });
                }
                // bf16 of block (c32, j) after the lane swaps: piece[h] holds
                // 16-byte chunk 2h + v of the block's 64 bytes in the lane's row
                auto block_bits = [&](auto C32, auto J, float fa, i32x4 (&piece)[2])
                    __attribute__((always_inline)) {
                    constexpr int c32 = decltype(C32)::value, j = decltype(J)::value;
                    uint32_t x[4][2];   // per q: bf16 pairs of columns 32j + 8q + 4v + {0,1} / {2,3}
                    static_for<4>([&](auto Q) {
                        constexpr int q = decltype(Q)::value;
                        float e[4];
                        static_for<4>([&](auto I) { e[decltype(I)::value] = acc[c32][j][4 * q + decltype(I)::value]; });
                        if constexpr (bz) {
                            const f32x4 f = fcol[j][q];
                            const uint32_t b0 = zw[j][q][0], b1 = zw[j][q][1];
                            const float z[4] = {bf16_lo(b0), bf16_hi(b0), bf16_lo(b1), bf16_hi(b1)};
                            static_for<4>([&](auto I) {
                                constexpr int i = decltype(I)::value;
                                e[i] = add_nc(e[i] * (fa * f[i]), z[i]);
                            });
                        } else if constexpr (hf) {
                            const f32x4 f = fcol[j][q];
                            static_for<4>([&](auto I) {
                                constexpr int i = decltype(I)::value;
                                e[i] = e[i] * (fa * f[i]);
                            });
                        }
                        x[q][0] = pack_bf16x2(e[0], e[1]);
                        x[q][1] = pack_bf16x2(e[2], e[3]);
                    });
                    // lanes 0-31 get columns 8q..8q+7, lanes 32-63 8(q+1)..8(q+1)+7
                    static_for<2>([&](auto H2) {
                        constexpr int q = 2 * decltype(H2)::value;
                        auto s0 = __builtin_amdgcn_permlane32_swap(x[q][0], x[q + 1][0], false, false);
                        auto s1 = __builtin_amdgcn_permlane32_swap(x[q][1], x[q + 1][1], false, false);
                        piece[decltype(H2)::value] = i32x4{(int)s0[0], (int)s1[0], (int)s0[1], (int)s1[1]};
                    });
                };
                // Jobs: per 32-row block c32, NL whole 128-byte lines and (odd
                // FN32) the trailing 64-byte block.  Software-pipelined by one
                // job: job k+1 is converted while job k's staging round trip
                // is in flight.
                constexpr int JPB = NL + (T::FN32 % 2);   // jobs per row block
                constexpr int NJ = T::FM32 * JPB;
                auto job_bits = [&](auto KJ, i32x4 (&pc)[4]) __attribute__((always_inline)) {
                    constexpr int kj = decltype(KJ)::value;
                    constexpr int c32 = kj / JPB, ln = kj % JPB;
                    float fa = 1.0f;
                    if constexpr (hf) fa = frowf[par][c32 * 32 + m];
                    i32x4 a[2], b[2];
                    if constexpr (ln < NL) {
                        block_bits(std::integral_constant<int, c32>{}, std::integral_constant<int, 2 * ln>{}, fa, a);
                        block_bits(std::integral_constant<int, c32>{}, std::integral_constant<int, 2 * ln + 1>{}, fa, b);
                        pc[2] = b[0];
                        pc[3] = b[1];
                    } else {
                        block_bits(std::integral_constant<int, c32>{}, std::integral_constant<int, T::FN32 - 1>{}, fa, a);
                    }
                    pc[0] = a[0];
                    pc[1] = a[1];
                };
                i32x4 pc[4];
                job_bits(std::integral_constant<int, 0>{}, pc);
                static_for<NJ>([&](auto KJ) {
                    constexpr int kj = decltype(KJ)::value;
                    constexpr int c32 = kj / JPB, ln = kj % JPB;
                    f32x4 xv[4];
                    int col;
                    if constexpr (ln < NL) {
                        // pieces: chunk 4jj + 2h + v of the line
                        static_for<2>([&](auto J2) {
                            static_for<2>([&](auto H2) {
                                constexpr int jj = decltype(J2)::value, h2 = decltype(H2)::value;
                                const int chunk = 4 * jj + 2 * h2 + v;
                                *reinterpret_cast<i32x4*>(stg + m * 128 + ((chunk ^ (m & 7)) * 16)) = pc[2 * jj + h2];
                            });
                        });
                        const int rr = lane >> 3, cc = lane & 7;
                        col = col_w + ln * 64 + cc * 8;   // N % 16 == 0
                        static_for<4>([&](auto Bk) {
                            const int r = rr + 8 * decltype(Bk)::value;
                            xv[decltype(Bk)::value] = *reinterpret_cast<const f32x4*>(stg + r * 128 + ((cc ^ (r & 7)) * 16));
                        });
                    } else {
                        static_for<2>([&](auto H2) {
                            const int chunk = 2 * decltype(H2)::value + v;
                            *reinterpret_cast<i32x4*>(stg + m * 64 + ((chunk ^ ((m >> 1) & 3)) * 16)) =
                                pc[decltype(H2)::value];
                        });
                        const int rr = lane >> 2, cc = lane & 3;
                        col = col_w + NL * 64 + cc * 8;
                        static_for<2>([&](auto Bk) {
                            const int r = rr + 16 * decltype(Bk)::value;
                            xv[decltype(Bk)::value] =
                                *reinterpret_cast<const f32x4*>(stg + r * 64 + ((cc ^ ((r >> 1) & 3)) * 16));
                        });
                    }
                    if constexpr (kj + 1 < NJ) job_bits(std::integral_constant<int, kj + 1>{}, pc);
                    if constexpr (ln < NL) {
                        const int rr = lane >> 3;
                        static_for<4>([&](auto Bk) {
                            const int r = rr + 8 * decltype(Bk)::value;
                            const uint32_t o = (uint32_t)(((c32 * 32 + r) * p.N + col) * 2);
                            store16(rO, col < p.N ? o : kOOB, xv[decltype(Bk)::value]);
                        });
                    } else {
                        const int rr = lane >> 2;
                        static_for<2>([&](auto Bk) {
                            const int r = rr + 16 * decltype(Bk)::value;
                            const uint32_t o = (uint32_t)(((c32 * 32 + r) * p.N + col) * 2);
                            store16(rO, col < p.N ? o : kOOB, xv[decltype(Bk)::value]);
                        });
                    }
                    __builtin_amdgcn_sched_barrier(0);
                });
            };
            epi32(std::integral_constant<bool, AFF != 0>{}, std::integral_constant<bool, AFF == 2>{});
            }
        }
        ph.mark(kPhEpi);
        par ^= 1;
        factor_dma(nxt, par);
        bias_dma(nxt, par);
        cur = nxt;
        nxt = unit_of(id + 2 * G);
        ocur = onxt;
        onxt = orig_of(nxt);
    }
    // The last unit prefetched dead stages into LDS and registers: let every
    // transfer land before the workgroup's LDS is released.
    ph.mark(kPhEpi);
    wait_vmcnt<0>();
    ph.mark(kPhEpi);
    ph.flush(p.phase);
}

// ======================================================================
// Skinny (decode) kernel: M <= 16*MT, MT in {1,2}
// ======================================================================
// A workgroup owns 16*NF rows of B (NF preshuffled 16-row fragments) and
// NWK waves; wave kw owns a contiguous, 256-K aligned chunk of the K
// stages and streams all NF fragments of it, so each A fragment it loads
// (from L2: A is shared by every workgroup) feeds NF MFMAs.  B is read
// once, with the non-temporal policy; up to U stages of B, A and scales
// are in flight per wave.  Waves reduce their partial tiles through LDS
// in a fixed order (deterministic), then the waves run the epilogue of the
// NF*MT output fragments.  NF = 1 covers half a 32-row scale group; NF =
// 2*G covers G whole groups (one B-scale dword per group and 256 K).
// XBF: A is bf16 [M, K] (row stride K) and is quantized to MXFP4 in
// registers: the MFMA's A operand of lane l (row l % 16, K bytes 16*(l/16)
// of a 128-K stage) is exactly one 32-element block, so each lane loads its
// block's 64 bytes, quantizes it with the rule of the quantizer kernel and
// builds the scale operand from the bytes it computes, the ones the shuffled
// scale layout would hold at the op_sel positions (row tile m, stage parity h
// -> byte m + 2h).  The products equal quantizing A first and running the
// XBF = 0 kernel on the same plan, bit for bit.  Every workgroup quantizes
// all of A, so the quantizer's VALU work is repeated per workgroup.  The
// compact forms (one row tile) quantize only the live rows' blocks: XBF = 2
// (M <= 4) in one pass, XBF = 3 (M <= 8) in two.  In pass q lane j takes
// block (row 4q + j/16, stage (j/4)%4, K-block j%4) of a 4-stage batch;
// ds_bpermute then moves codes and scale bytes to the MFMA lanes.
// XMBS (compact forms, no K split): MBS activations.  Every workgroup first
// takes each row's maximum over all of K (its waves split K, then reduce
// through LDS), derives the row's factor byte as the MBS quantizer does, and
// quantizes the row times 1 + b/256; the epilogue applies f(b) with the B
// factors (p.Bf) as the factor GEMM does with a stored A factor.
template <int MT, int NF, int NWK, int U, bool SPLIT, int XBF = 0, bool XMBS = false>
__global__ void __launch_bounds__(64 * NWK) gemm_skinny_kernel(const GemmArgs p)
{
    static_assert(U % 2 == 0, "batch must cover whole 256-K scale groups");
    static_assert(NF == 1 || NF % 2 == 0, "whole 32-row scale groups (or half of one)");
    constexpr int NG = (NF + 1) / 2;   // 32-row B-scale groups per workgroup
    // Stages per batch.  XBF holds 16 registers of bf16 A per stage and row
    // tile: at 4 waves per SIMD (128 registers a wave) the batch is cut to
    // 4 fragments of A so nothing spills.  The accumulation order over the
    // stages does not depend on the batch.
    constexpr int UB = (XBF && NWK >= 8 && MT * U > 4) ? 4 / MT : U;
    constexpr bool XC = XBF >= 2;
    constexpr int NP = XC ? XBF - 1 : 1;   // compact passes: 4 rows each
    static_assert(!XC || (MT == 1 && UB == 4 && NP <= 2), "compact bf16 A: one row tile, 4-stage batches");
    static_assert(!XMBS || (XC && !SPLIT), "MBS activations: compact forms, whole K");
    __shared__ f32x4 red[NWK][NF * MT][64];
    __shared__ uint32_t row_max[XMBS ? NWK : 1][8];
    __shared__ uint32_t row_fb[16];   // rows 8..15 (past M) stay 0

    const int lane = threadIdx.x & 63;
    const int kw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * 16 * NF;
    const int split = blockIdx.y;

    const int K = p.K, Kp = K >> 1;
    const int S_total = (K + 127) >> 7;
    const int s_begin = split * p.sps;
    const int s_end = min(s_begin + p.sps, S_total);
    const int n_st = s_end - s_begin;
    const int CH = (((n_st + NWK - 1) / NWK) + 1) & ~1;
    const int my_begin = s_begin + kw * CH;
    const int my_end = min(my_begin + CH, s_end);

    // B fragments beyond N read as zeros (range = valid fragments only).
    const int nfrag = min(NF, (p.N - n0) >> 4);
    const uint32_t fstride = (uint32_t)K * 8;  // bytes of one 16-row fragment column
    const rsrc_t rB = make_rsrc(p.B + (size_t)(n0 >> 4) * fstride, (uint32_t)nfrag * fstride);
    // bf16 A (XBF): rows >= M read as zeros from outside the range
    const rsrc_t rA = make_rsrc(p.A, (uint32_t)(p.M * (XBF ? 2 * K : Kp)));
    const rsrc_t rAs = make_rsrc(p.As, XBF ? 0u : (uint32_t)(32 * p.snp));
    const int Npad = (p.N + 31) & ~31;
    const rsrc_t rBs = make_rsrc(p.Bs + (size_t)(n0 >> 5) * 32 * p.snp,
                                 (uint32_t)(min(NG * 32, Npad - ((n0 >> 5) << 5)) * p.snp));
    const bool hi_lane = lane >= 32;
    const bool ktail = (K & 127) != 0;
    // NF == 1: the workgroup's 16 rows are the low or high half of a 32-row
    // scale group; shift that half's bytes into the op_sel 0/2 positions.
    const int sshift = NF == 1 ? 8 * ((n0 >> 4) & 1) : 0;

    f32x4 acc[NF][MT];
    static_for<NF>([&](auto f) {
        static_for<MT>([&](auto m) { acc[f][m] = f32x4{0.f, 0.f, 0.f, 0.f}; });
    });

    // Scale dwords and B fragments of the batch starting at stage st.
    auto issue_b = [&](int st, i32x4 (&b)[UB][NF], int (&sb)[UB / 2][NG]) {
        static_for<UB / 2>([&](auto v) {
            const int g = (st >> 1) + v;
            const bool ok = st + 2 * v < my_end;
            static_for<NG>([&](auto G) {
                sb[v][G] = load4(rBs, ok ? (uint32_t)(G * 32 * p.snp + g * 256 + lane * 4) : kOOB);
            });
        });
        static_for<UB>([&](auto u) {
            const int s = st + u;
            const bool zap = (ktail && s == S_total - 1 && hi_lane) || s >= my_end;
            static_for<NF>([&](auto f) {
                b[u][f] = load16nt(rB, zap ? kOOB : (uint32_t)(f * fstride + s * 1024 + lane * 16));
            });
        });
    };
    float mrow[NP];   // XMBS: the multiplier 1 + b/256 of each pass's row
    // XMBS, one pass: the first PA chunks of every row go out first, then the
    // first batch's B; the row maxima wait for those chunks only (loads
    // return in issue order), and the barriers wait for LDS only, so the B
    // batch streams during the maximum pass.
    constexpr bool PRE_B = XMBS && NP == 1;
    constexpr int PA = 2;
    i32x4 b_first[PRE_B ? UB : 1][NF];
    int sb_first[PRE_B ? UB / 2 : 1][NG];
    if constexpr (XMBS) {
        constexpr int NR = 4 * NP;   // rows >= M read zeros
        const int e0 = (kw * 64 + lane) * 8;
        i32x4 a0[NR][PA];
        static_for<NR>([&](auto r) {
            static_for<PA>([&](auto j) {
                const int e = e0 + j * NWK * 512;
                a0[r][j] = load16(rA, e < K ? (uint32_t)((r * K + e) * 2) : kOOB);
            });
        });
        if constexpr (PRE_B) issue_b(my_begin, b_first, sb_first);
        static_for<NR>([&](auto r) {
            uint32_t amax = 0;
            static_for<PA>([&](auto j) { amax = max(amax, bf16x8_absmax(a0[r][j])); });
            for (int e = e0 + PA * NWK * 512; e < K; e += NWK * 512)
                amax = max(amax, bf16x8_absmax(load16(rA, (uint32_t)((r * K + e) * 2))));
            for (int off = 32; off >= 1; off >>= 1) amax = max(amax, (uint32_t)__shfl_xor((int)amax, off));
            if (lane == 0) row_max[kw][r] = amax;
        });
        wait_lgkmcnt0();
        barrier();
        if (threadIdx.x < 16) {
            uint32_t amax = 0;
            if (threadIdx.x < NR)
                for (int k = 0; k < NWK; ++k) amax = max(amax, row_max[k][threadIdx.x]);
            row_fb[threadIdx.x] = mbs_factor_byte(amax);
        }
        wait_lgkmcnt0();
        barrier();
        static_for<NP>([&](auto q) {
            mrow[q] = __uint_as_float(0x3F800000u | (row_fb[4 * q + (lane >> 4)] << 15));
        });
    }

    for (int st = my_begin; st < my_end; st += UB) {
        i32x4 b[UB][NF], a[UB][MT];
        int sb[UB / 2][NG], sa[UB / 2];
        i32x4 x[XBF == 1 ? UB : 1][XBF == 1 ? MT : 1][4];  // XBF 1: the lane's bf16 A blocks
        i32x4 xc[NP][4];   // compact: block (row 4q + lane/16, stage (lane/4)%4, K-block lane%4)
        if constexpr (XC) {
            // first in the issue order: the quantization then waits for these
            // (from L2) and not for the batch's B stream; rows >= M lie
            // outside the range and read as zeros
            const int s = st + ((lane >> 2) & 3), kb = lane & 3;
            const bool zap = (ktail && s == S_total - 1 && kb >= 2) || s >= my_end;
            static_for<NP>([&](auto q) {
                const uint32_t o = (uint32_t)(((4 * q + (lane >> 4)) * K + s * 128 + kb * 32) * 2);
                static_for<4>([&](auto i) { xc[q][i] = load16(rA, zap ? kOOB : o + 16 * i); });
            });
        }
        // Scales first: loads return in issue order, so stage u's MFMAs then
        // wait only for stage u's B and A, and the MFMAs trail the stream
        // instead of starting after the whole batch has landed.
        if constexpr (PRE_B) {
            if (st == my_begin) {
                static_for<UB>([&](auto u) { static_for<NF>([&](auto f) { b[u][f] = b_first[u][f]; }); });
                static_for<UB / 2>([&](auto v) { static_for<NG>([&](auto G) { sb[v][G] = sb_first[v][G]; }); });
            } else {
                issue_b(st, b, sb);
            }
        } else {
            static_for<UB / 2>([&](auto v) {
                const int g = (st >> 1) + v;
                const bool ok = st + 2 * v < my_end;
                static_for<NG>([&](auto G) {
                    sb[v][G] = load4(rBs, ok ? (uint32_t)(G * 32 * p.snp + g * 256 + lane * 4) : kOOB);
                });
                if constexpr (!XBF) sa[v] = load4(rAs, ok ? (uint32_t)(g * 256 + lane * 4) : kOOB);
            });
            static_for<UB>([&](auto u) {
                const int s = st + u;
                const bool ok = s < my_end;
                const bool zap = (ktail && s == S_total - 1 && hi_lane) || !ok;
                static_for<NF>([&](auto f) {
                    b[u][f] = load16nt(rB, zap ? kOOB : (uint32_t)(f * fstride + s * 1024 + lane * 16));
                });
                static_for<MT>([&](auto m) {
                    if constexpr (XC) {
                    } else if constexpr (XBF) {
                        // a row tile wholly past M reads nothing (and is not quantized)
                        const bool dead = zap || 16 * m >= p.M;
                        const uint32_t o = (uint32_t)(((16 * m + (lane & 15)) * K + s * 128 + (lane >> 4) * 32) * 2);
                        static_for<4>([&](auto i) { x[u][m][i] = load16(rA, dead ? kOOB : o + 16 * i); });
                    } else {
                        a[u][m] = load16(rA, zap ? kOOB
                                                 : (uint32_t)((16 * m + (lane & 15)) * Kp + s * 64 +
                                                              (lane >> 4) * 16));
                    }
                });
            });
        }
        // Every load of the batch is issued before the first MFMA; left to
        // itself the scheduler interleaves them with the MFMAs and the wave
        // keeps only a fraction of its batch in flight.
        __builtin_amdgcn_sched_barrier(0);
        i32x4 qc[NP];
        uint32_t qe[NP] = {};
        if constexpr (XMBS) static_for<NP>([&](auto q) { qc[q] = quantize_block32_mbs(xc[q], mrow[q], &qe[q]); });
        else if constexpr (XC) static_for<NP>([&](auto q) { qc[q] = quantize_block32(xc[q], &qe[q]); });
        static_for<UB>([&](auto u) {
            constexpr int h = u & 1;
            const int s = st + u;
            const bool tail = ktail && s == S_total - 1 && hi_lane;
            int sav;
            if constexpr (XC) {
                // MFMA lane (row r = l%16, K-block l/16) <- pass r/4, lane
                // 16*(r%4) + 4u + l/16; rows from 4*NP on are past M
                const int r = lane & 15;
                const bool live = r < 4 * NP;
                const int src = ((r & 3) * 16 + 4 * u + (lane >> 4)) * 4;
                static_for<4>([&](auto i) {
                    constexpr int I = decltype(i)::value;
                    int v = __builtin_amdgcn_ds_bpermute(src, qc[0][I]);
                    if constexpr (NP == 2) {
                        const int v1 = __builtin_amdgcn_ds_bpermute(src, qc[1][I]);
                        v = r >= 4 ? v1 : v;
                    }
                    a[u][0][I] = live ? v : 0;
                });
                uint32_t e = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)qe[0]);
                if constexpr (NP == 2) {
                    const uint32_t e1 = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)qe[1]);
                    e = r >= 4 ? e1 : e;
                }
                sav = live ? (int)(e << (16 * h)) : 0;
            } else if constexpr (XBF) {
                // this stage's blocks: codes into a[u][m], scales to byte m + 2h
                uint32_t sq = 0;
                static_for<MT>([&](auto m) {
                    uint32_t e = 0;
                    if (16 * m < p.M) a[u][m] = quantize_block32(x[u][m], &e);
                    else a[u][m] = i32x4{0, 0, 0, 0};
                    sq |= e << (8 * (m + 2 * h));
                });
                sav = (int)sq;
            } else {
                sav = sa[u / 2];
            }
            sav = tail ? 0x7F7F7F7F : sav;
            static_for<NF>([&](auto f) {
                int sbv = sb[u / 2][f / 2] >> sshift;
                sbv = tail ? 0x7F7F7F7F : sbv;
                static_for<MT>([&](auto m) {
                    mfma_fp4<(f & 1) + 2 * h, m + 2 * h>(acc[f][m], b[u][f], a[u][m], sbv, sav);
                });
            });
        });
    }

    mfma_drain();
    static_for<NF>([&](auto f) {
        static_for<MT>([&](auto m) { pin_after_drain(acc[f][m]); });
    });
    static_for<NF>([&](auto f) {
        static_for<MT>([&](auto m) { red[kw][f * MT + m][lane] = acc[f][m]; });
    });
    __syncthreads();
    // output fragment o = f * MT + m, handled by wave o % NWK
    for (int o = kw; o < NF * MT; o += NWK) {
        const int f = o / MT, m = o % MT;
        if (n0 + 16 * f >= p.N) continue;
        f32x4 v = red[0][o][lane];
        for (int k = 1; k < NWK; ++k) v += red[k][o][lane];
        const int c = n0 + 16 * f + (lane >> 4) * 4;
        const int row = 16 * m + (lane & 15);
        if constexpr (SPLIT) {
            const rsrc_t rW = make_rsrc(p.ws + (size_t)split * p.M * p.N, (uint32_t)(p.M * p.N * 4));
            store16(rW, (uint32_t)((row * p.N + c) * 4), v);
        } else {
            if (XMBS || (p.Af && p.Bf)) {
                const rsrc_t rAf = make_rsrc(p.Af, XMBS ? 0u : (uint32_t)p.M);
                const rsrc_t rBf = make_rsrc(p.Bf, (uint32_t)p.N);
                const uint32_t ab = XMBS ? row_fb[row] : load1(rAf, row);
                const float fa = factor_of(ab) * p.alpha;
                const uint32_t bytes = (uint32_t)load4(rBf, c);
                for (int q = 0; q < 4; ++q) v[q] = v[q] * (fa * factor_of(bytes >> (8 * q)));
            } else if (p.alpha != 1.0f) {
                for (int q = 0; q < 4; ++q) v[q] = v[q] * p.alpha;
            }
            if (p.bias) {
                const rsrc_t rBias = make_rsrc(p.bias, (uint32_t)(p.N * 2));
                const i32x2 bw = load8(rBias, (uint32_t)(c * 2));
                v[0] = add_nc(v[0], bf16_lo((uint32_t)bw[0])); v[1] = add_nc(v[1], bf16_hi((uint32_t)bw[0]));
                v[2] = add_nc(v[2], bf16_lo((uint32_t)bw[1])); v[3] = add_nc(v[3], bf16_hi((uint32_t)bw[1]));
            }
            const rsrc_t rO = make_rsrc(p.out, (uint32_t)(p.M * p.N * 2));
            store8(rO, (uint32_t)((row * p.N + c) * 2), pack_bf16x2(v[0], v[1]),
                   pack_bf16x2(v[2], v[3]));
        }
    }
}

// A non-split launch of the persistent kernel in the epilogue form the
// arguments ask for.
template <class T, bool GEN, bool GROUPED>
void launch_bdirect_form(const GemmArgs& a, dim3 grid, hipStream_t s)
{
    switch (epilogue_form(a)) {
    case 2: hipLaunchKernelGGL((gemm_bdirect_kernel<T, GEN, false, GROUPED, 2>), grid, dim3(T::NT), 0, s, a); break;
    case 1: hipLaunchKernelGGL((gemm_bdirect_kernel<T, GEN, false, GROUPED, 1>), grid, dim3(T::NT), 0, s, a); break;
    default: hipLaunchKernelGGL((gemm_bdirect_kernel<T, GEN, false, GROUPED, 0>), grid, dim3(T::NT), 0, s, a);
    }
}

template <class T>
hipError_t launch_bdirect(const GemmArgs& a, dim3 grid, bool gen, bool split, hipStream_t s)
{
    if constexpr (T::M32) {
        // whole-K, single-split plans only (make_plan offers no other)
        if (gen || split) return hipErrorInvalidValue;
        launch_bdirect_form<T, false, false>(a, grid, s);
    } else if (gen) {
        if (split) hipLaunchKernelGGL((gemm_bdirect_kernel<T, true, true>), grid, dim3(T::NT), 0, s, a);
        else launch_bdirect_form<T, true, false>(a, grid, s);
    } else {
        if (split) hipLaunchKernelGGL((gemm_bdirect_kernel<T, false, true>), grid, dim3(T::NT), 0, s, a);
        else launch_bdirect_form<T, false, false>(a, grid, s);
    }
    return hipGetLastError();
}

// Grouped (MoE) launches of the persistent kernel (no K splits).
template <class T>
hipError_t launch_bdirect_grouped(const GemmArgs& a, dim3 grid, bool gen, bool, hipStream_t s)
{
    if constexpr (T::M32) {
        // whole-K plans only (run_grouped refuses K % 512 != 0)
        if (gen) return hipErrorInvalidValue;
        launch_bdirect_form<T, false, true>(a, grid, s);
    } else if (gen) {
        launch_bdirect_form<T, true, true>(a, grid, s);
    } else {
        launch_bdirect_form<T, false, true>(a, grid, s);
    }
    return hipGetLastError();
}

template <int MT, int NF, int NWK, int U>
hipError_t launch_skinny(const GemmArgs& a, dim3 grid, bool, bool split, hipStream_t s)
{
    if (split) hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, true>), grid, dim3(64 * NWK), 0, s, a);
    else hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, false>), grid, dim3(64 * NWK), 0, s, a);
    return hipGetLastError();
}

// The same plans with A given as bf16 and quantized in registers; one row
// tile with M <= 8 takes a compact form.
template <int MT, int NF, int NWK, int U>
hipError_t launch_skinny_xbf(const GemmArgs& a, dim3 grid, bool, bool split, hipStream_t s)
{
    if constexpr (MT == 1) {
        // MBS activations (B factors given, the A factors derived in the
        // kernel): compact forms without a K split only
        if (a.Bf) {
            if (split || a.M > 8) return hipErrorInvalidValue;
            if (a.M <= 4) hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, false, 2, true>), grid, dim3(64 * NWK), 0, s, a);
            else hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, false, 3, true>), grid, dim3(64 * NWK), 0, s, a);
            return hipGetLastError();
        }
        if (a.M <= 4) {
            if (split) hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, true, 2>), grid, dim3(64 * NWK), 0, s, a);
            else hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, false, 2>), grid, dim3(64 * NWK), 0, s, a);
            return hipGetLastError();
        }
        if (a.M <= 8) {
            if (split) hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, true, 3>), grid, dim3(64 * NWK), 0, s, a);
            else hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, false, 3>), grid, dim3(64 * NWK), 0, s, a);
            return hipGetLastError();
        }
    }
    if (a.Bf) return hipErrorInvalidValue;
    if (split) hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, true, 1>), grid, dim3(64 * NWK), 0, s, a);
    else hipLaunchKernelGGL((gemm_skinny_kernel<MT, NF, NWK, U, false, 1>), grid, dim3(64 * NWK), 0, s, a);
    return hipGetLastError();
}

using B256x256 = BdShape<256, 256, 2, 2>;
using B256x128 = BdShape<256, 128, 2, 2>;
using B128x256 = BdShape<128, 256, 2, 2>;
using B128x128 = BdShape<128, 128, 2, 2>;
using B64x256 = BdShape<64, 256, 1, 4>;
using B64x128 = BdShape<64, 128, 1, 2>;
using B64x64 = BdShape<64, 64, 1, 1>;
using B256x256w14 = BdShape<256, 256, 1, 4>;
using B192x256w14 = BdShape<192, 256, 1, 4>;
using B96x256w14 = BdShape<96, 256, 1, 4>;
using B64x512w14 = BdShape<64, 512, 1, 4>;
using B128x384w14 = BdShape<128, 384, 1, 4>;
using B256x128w14 = BdShape<256, 128, 1, 4>;
using B128x256w14 = BdShape<128, 256, 1, 4>;
// 32x32x64 MFMA tiles
using B96x256m = BdShape<96, 256, 1, 4, true>;
using B128x256m = BdShape<128, 256, 1, 4, true>;
using B192x256m = BdShape<192, 256, 1, 4, true>;
using B256x256m = BdShape<256, 256, 1, 4, true>;
using B128x384m = BdShape<128, 384, 1, 4, true>;


// Launcher instantiations, one translation unit per group (gemm_inst_*.hip).
#define MBS_BDIRECT_SHAPES_A(X) X(B256x256) X(B256x128) X(B128x256) X(B128x128)
#define MBS_BDIRECT_SHAPES_B(X) X(B64x256) X(B64x128) X(B64x64) X(B256x128w14)
#define MBS_BDIRECT_SHAPES_C(X) X(B256x256w14) X(B192x256w14) X(B96x256w14)
#define MBS_BDIRECT_SHAPES_D(X) X(B64x512w14) X(B128x384w14) X(B128x256w14)
#define MBS_BDIRECT_SHAPES_E(X) X(B96x256m) X(B128x256m) X(B192x256m) X(B256x256m) X(B128x384m)
#define MBS_GROUPED_SHAPES(X) X(B256x256) X(B128x256w14) X(B64x256) X(B64x128)
#define MBS_GROUPED_SHAPES_M(X) X(B128x256m) X(B256x256m)
#define MBS_SKINNY_SHAPES(X) X(1, 2, 16, 4) X(2, 2, 16, 4) X(1, 2, 8, 4) X(2, 2, 8, 4) X(1, 1, 8, 8) X(2, 1, 8, 8) X(2, 2, 4, 4)

#define MBS_LAUNCH_SIG const GemmArgs&, dim3, bool, bool, hipStream_t
#define MBS_BDIRECT_INST(T) template hipError_t launch_bdirect<T>(MBS_LAUNCH_SIG);
#define MBS_SKINNY_INST(a, b, c, d)                                 \
    template hipError_t launch_skinny<a, b, c, d>(MBS_LAUNCH_SIG); \
    template hipError_t launch_skinny_xbf<a, b, c, d>(MBS_LAUNCH_SIG);
#define MBS_GROUPED_INST(T) template hipError_t launch_bdirect_grouped<T>(MBS_LAUNCH_SIG);
#define MBS_GROUPED_EXTERN(T) extern template hipError_t launch_bdirect_grouped<T>(MBS_LAUNCH_SIG);
#define MBS_BDIRECT_EXTERN(T) extern template hipError_t launch_bdirect<T>(MBS_LAUNCH_SIG);
#define MBS_SKINNY_EXTERN(a, b, c, d)                                     \
    extern template hipError_t launch_skinny<a, b, c, d>(MBS_LAUNCH_SIG); \
    extern template hipError_t launch_skinny_xbf<a, b, c, d>(MBS_LAUNCH_SIG);

}  // namespace mbs
