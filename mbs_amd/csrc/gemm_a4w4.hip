// MXFP4 A4W4 GEMM for MI355X (gfx950):  out[M,N] (bf16) =
//   (dequant(A) . dequant(B)^T) * f(AFactor)[m] * f(BFactor)[n],  fp32 accumulate.
//
// Operand bytes follow the reference's contract (kernel/gemm_a4w4.h:5-26 of
// the reference): plain row-major A [M,K/2], (16,16)-preshuffled B, shuffled
// E8M0 scales.  Kernel families (gemm_kernels.h):
//
//  * gemm_bdirect_kernel -- persistent workgroups (one resident set per CU)
//    loop over BM x BN tiles (x K-splits) in an XCD-aware order.  A moves
//    global->LDS by 16-byte buffer_load ... lds DMA in 256-K pairs of whole
//    cache lines, XOR-swizzled so the MFMA fragment reads are conflict-free;
//    the preshuffled B is already in fragment order and loads straight into
//    a VGPR ring.  The MFMA is issued with the operands swapped (B as src0)
//    so each lane owns 4 consecutive n of one output row; the epilogue
//    applies the MBS factors / alpha / bias, packs bf16 (RNE) and stores 16
//    bytes per lane after two rounds of lane swaps.
//  * gemm_skinny_kernel -- decode shapes (M <= 32): each wave streams 16 or
//    32 rows of B (non-temporal) straight into VGPRs with a batch of its
//    K-chunk in flight, reusing each A fragment for every B fragment; waves
//    of a workgroup split K and reduce through LDS in a fixed order.  Its
//    bf16-activation form quantizes A in registers (one launch from a bf16
//    activation, mbs_gemm_a4w4_from_bf16_launch).
//  * splitk_reduce_kernel -- deterministic fixed-order sum of fp32 split-K
//    partials plus the same epilogue.
#include "gemm_kernels.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

namespace mbs {

// Scratch of the allocation-free entry point (mbs_gemm_a4w4_launch_noalloc):
// its split-K partials live here instead of in a caller workspace.  Each GPU
// the library runs on holds its own copy until the process ends.  In host
// code `scratch` is only a symbol handle; its address on a device comes from
// hipGetSymbolAddress with that device current (scratch_on_current_device).
static __device__ __align__(256) uint8_t scratch[MBS_NOALLOC_SCRATCH_BYTES];

namespace {
thread_local std::string g_last_error;
// Phase-timer sums the persistent kernels add into (timer builds only).
unsigned long long* g_phase = nullptr;
}
void set_last_error(const char* msg) { g_last_error = msg ? msg : ""; }

MBS_BDIRECT_SHAPES_A(MBS_BDIRECT_EXTERN)
MBS_BDIRECT_SHAPES_B(MBS_BDIRECT_EXTERN)
MBS_BDIRECT_SHAPES_C(MBS_BDIRECT_EXTERN)
MBS_BDIRECT_SHAPES_D(MBS_BDIRECT_EXTERN)
MBS_BDIRECT_SHAPES_E(MBS_BDIRECT_EXTERN)
MBS_SKINNY_SHAPES(MBS_SKINNY_EXTERN)
MBS_GROUPED_SHAPES(MBS_GROUPED_EXTERN)
MBS_GROUPED_SHAPES_M(MBS_GROUPED_EXTERN)

// ======================================================================
// Split-K reduction: out[m][n..n+3] = epilogue(sum_s ws[s][m][n..n+3])
// ======================================================================
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const GemmArgs p)
{
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int nq = p.N >> 2;
    if (q >= (int64_t)p.M * nq) return;
    const int m = (int)(q / nq);
    const int c = (int)(q - (int64_t)m * nq) * 4;
    const size_t plane = (size_t)p.M * p.N;
    const f32x4* src = reinterpret_cast<const f32x4*>(p.ws + (size_t)m * p.N + c);
    f32x4 v = src[0];
    for (int s = 1; s < p.splits; ++s) v += *reinterpret_cast<const f32x4*>(p.ws + s * plane + (size_t)m * p.N + c);
    if (p.Af && p.Bf) {
        const float fa = factor_of(p.Af[m]) * p.alpha;
        const uint32_t bytes = *reinterpret_cast<const uint32_t*>(p.Bf + c);
        for (int k = 0; k < 4; ++k) v[k] = v[k] * (fa * factor_of(bytes >> (8 * k)));
    } else if (p.alpha != 1.0f) {
        for (int k = 0; k < 4; ++k) v[k] = v[k] * p.alpha;
    }
    if (p.bias) {
        const uint32_t* bw = reinterpret_cast<const uint32_t*>(p.bias + c);
        v[0] = add_nc(v[0], bf16_lo(bw[0])); v[1] = add_nc(v[1], bf16_hi(bw[0]));
        v[2] = add_nc(v[2], bf16_lo(bw[1])); v[3] = add_nc(v[3], bf16_hi(bw[1]));
    }
    uint32_t* o = reinterpret_cast<uint32_t*>(p.out + (size_t)m * p.N + c);
    o[0] = pack_bf16x2(v[0], v[1]);
    o[1] = pack_bf16x2(v[2], v[3]);
}

// ======================================================================
// Expert-offset report of a grouped launch (one workgroup):
//   status[0] = non-empty experts whose first row is not a multiple of 32
//               (the grouped kernel skips them: their rows are not written),
//   status[1] = offsets the kernel clamps: offsets[0] != 0, an entry outside
//               [0, M], or a decrease offsets[e+1] < offsets[e].
// ======================================================================
__global__ void __launch_bounds__(256) check_groups_kernel(const int* off, int E, int M, uint32_t* status)
{
    __shared__ uint32_t cnt[2];
    if (threadIdx.x < 2) cnt[threadIdx.x] = 0;
    __syncthreads();
    uint32_t unaligned = 0, clamped = 0;
    for (int e = threadIdx.x; e <= E; e += 256) {
        const int v = off[e];
        clamped += (v < 0 || v > M || (e == 0 && v != 0) || (e < E && off[e + 1] < v)) ? 1u : 0u;
        if (e < E) {
            const int b = min(max(v, 0), M), end = min(max(off[e + 1], b), M);
            unaligned += (end > b && (b & 31) != 0) ? 1u : 0u;
        }
    }
    atomicAdd(&cnt[0], unaligned);
    atomicAdd(&cnt[1], clamped);
    __syncthreads();
    if (threadIdx.x < 2) status[threadIdx.x] = cnt[threadIdx.x];
}

// ======================================================================
// Host side: configurations, plans, launch
// ======================================================================
namespace {

int fail(int code, const std::string& msg)
{
    set_last_error(msg.c_str());
    return code;
}

enum Family { kPersistent = 0, kSkinny = 1 };

struct Config {
    const char* name;
    Family family;
    int bm, bn;        // persistent: workgroup tile; skinny: rows covered (16*MT) x B rows (16*NF)
    int threads;
    int wgs_per_cu;    // resident workgroups per CU (LDS / register bound)
    // Cost model constants.  Persistent: {us per 128-K stage with one workgroup
    // on the CU, us per stage with wgs_per_cu of them, us per work unit},
    // fitted to graph-replayed timings of every config and split count on 22
    // shapes on MI355X.  Skinny: {streaming efficiency, 0, 0}.
    struct {
        float a, b, c;
    } cost;
    // launch(args, grid, general, split, stream); general: the dead-stage /
    // K-tail variant
    hipError_t (*launch)(const GemmArgs&, dim3, bool, bool, hipStream_t);
    bool persistent = false;  // grid capped at the resident slots; workgroups loop over units
    // whole K only: no K tail, no dead stages (K % 512 == 0), one split
    // (the 32x32x64 MFMA tiles)
    bool whole_k = false;
    // skinny: the same plan with A given as bf16, quantized in registers
    hipError_t (*launch_xbf)(const GemmArgs&, dim3, bool, bool, hipStream_t) = nullptr;
};

const Config kConfigs[] = {
    {"bdirect_256x256_w2x2", kPersistent, 256, 256, 256, 1, {0.612f, 0.612f, 6.57f}, launch_bdirect<B256x256>, true},
    {"bdirect_256x128_w2x2", kPersistent, 256, 128, 256, 1, {0.389f, 0.389f, 3.09f}, launch_bdirect<B256x128>, true},
    {"bdirect_128x256_w2x2", kPersistent, 128, 256, 256, 1, {0.415f, 0.415f, 3.38f}, launch_bdirect<B128x256>, true},
    {"bdirect_128x128_w2x2", kPersistent, 128, 128, 256, 2, {0.235f, 0.446f, 2.54f}, launch_bdirect<B128x128>, true},
    {"bdirect_64x256_w1x4", kPersistent, 64, 256, 256, 2, {0.235f, 0.434f, 2.40f}, launch_bdirect<B64x256>, true},
    {"bdirect_64x128_w1x2", kPersistent, 64, 128, 128, 3, {0.191f, 0.357f, 1.96f}, launch_bdirect<B64x128>, true},
    {"bdirect_64x64_w1x1", kPersistent, 64, 64, 64, 4, {0.198f, 0.274f, 1.59f}, launch_bdirect<B64x64>, true},
    {"bdirect_256x256_w1x4", kPersistent, 256, 256, 256, 1, {0.611f, 0.611f, 7.01f}, launch_bdirect<B256x256w14>, true},
    {"bdirect_256x128_w1x4", kPersistent, 256, 128, 256, 1, {0.383f, 0.383f, 3.03f}, launch_bdirect<B256x128w14>, true},
    {"bdirect_128x256_w1x4", kPersistent, 128, 256, 256, 1, {0.367f, 0.367f, 3.14f}, launch_bdirect<B128x256w14>, true},
    {"bdirect_192x256_w1x4", kPersistent, 192, 256, 256, 1, {0.467f, 0.467f, 4.17f}, launch_bdirect<B192x256w14>, true},
    {"bdirect_96x256_w1x4", kPersistent, 96, 256, 256, 1, {0.290f, 0.290f, 2.77f}, launch_bdirect<B96x256w14>, true},
    {"bdirect_64x512_w1x4", kPersistent, 64, 512, 256, 1, {0.428f, 0.428f, 3.26f}, launch_bdirect<B64x512w14>, true},
    {"bdirect_128x384_w1x4", kPersistent, 128, 384, 256, 1, {0.455f, 0.455f, 4.55f}, launch_bdirect<B128x384w14>, true},
    // v_mfma_scale_f32_32x32x64_f8f6f4 tiles
    {"bdirect_96x256_w1x4_m32", kPersistent, 96, 256, 256, 1, {0.333f, 0.333f, 2.77f}, launch_bdirect<B96x256m>, true, true},
    {"bdirect_128x256_w1x4_m32", kPersistent, 128, 256, 256, 1, {0.367f, 0.367f, 3.14f}, launch_bdirect<B128x256m>, true, true},
    {"bdirect_192x256_w1x4_m32", kPersistent, 192, 256, 256, 1, {0.467f, 0.467f, 4.17f}, launch_bdirect<B192x256m>, true, true},
    {"bdirect_256x256_w1x4_m32", kPersistent, 256, 256, 256, 1, {0.611f, 0.611f, 7.01f}, launch_bdirect<B256x256m>, true, true},
    {"bdirect_128x384_w1x4_m32", kPersistent, 128, 384, 256, 1, {0.455f, 0.455f, 4.55f}, launch_bdirect<B128x384m>, true, true},
    // skinny: bm = rows covered (16*MT), bn = B rows per workgroup (16*NF)
    // eff = streaming efficiency relative to the best variant (cold N=K=8192 timings)
    {"skinny_m16_n32_w16", kSkinny, 16, 32, 1024, 1, {0.94f, 0.f, 0.f}, launch_skinny<1, 2, 16, 4>, false, false, launch_skinny_xbf<1, 2, 16, 4>},
    {"skinny_m32_n32_w16", kSkinny, 32, 32, 1024, 1, {0.89f, 0.f, 0.f}, launch_skinny<2, 2, 16, 4>, false, false, launch_skinny_xbf<2, 2, 16, 4>},
    {"skinny_m16_n32_w8", kSkinny, 16, 32, 512, 2, {1.00f, 0.f, 0.f}, launch_skinny<1, 2, 8, 4>, false, false, launch_skinny_xbf<1, 2, 8, 4>},
    {"skinny_m32_n32_w8", kSkinny, 32, 32, 512, 2, {0.92f, 0.f, 0.f}, launch_skinny<2, 2, 8, 4>, false, false, launch_skinny_xbf<2, 2, 8, 4>},
    {"skinny_m16_n16_w8", kSkinny, 16, 16, 512, 2, {0.91f, 0.f, 0.f}, launch_skinny<1, 1, 8, 8>, false, false, launch_skinny_xbf<1, 1, 8, 8>},
    {"skinny_m32_n16_w8", kSkinny, 32, 16, 512, 2, {0.69f, 0.f, 0.f}, launch_skinny<2, 1, 8, 8>, false, false, launch_skinny_xbf<2, 1, 8, 8>},
    {"skinny_m32_n32_w4", kSkinny, 32, 32, 256, 2, {1.00f, 0.f, 0.f}, launch_skinny<2, 2, 4, 4>, false, false, launch_skinny_xbf<2, 2, 4, 4>},
};
constexpr int kNumConfigs = (int)(sizeof(kConfigs) / sizeof(kConfigs[0]));
constexpr int kNumCUs = 256;

struct Plan {
    int config;
    int splits;
    int sps;
    dim3 grid;
    size_t ws_bytes;
};

int stages_of(int K) { return (K + 127) / 128; }

// Split count -> stages per split (even) and the realised split count.
void split_stages(int K, int want, int* sps, int* splits)
{
    const int S = stages_of(K);
    int per = (S + want - 1) / want;
    per = (per + 1) & ~1;
    if (per < 2) per = 2;
    *sps = per;
    *splits = (S + per - 1) / per;
}

double plan_cost(const Plan& pl, int M, int N, int K);

// Streaming waves per CU a skinny configuration needs to reach its measured
// rate: one workgroup per CU, at most 8 waves (timed cold at N=K=8192, the
// 4-wave M=32 variant with one workgroup per CU was the fastest M=32 plan).
int skinny_waves_per_cu(const Config& c) { return std::min(8, c.threads / 64); }

bool make_plan(int config, int want_splits, int M, int N, int K, Plan* out)
{
    if (config < 0 || config >= kNumConfigs) return false;
    const Config& c = kConfigs[config];
    Plan pl{};
    pl.config = config;
    if (c.family == kSkinny) {
        if (M > c.bm) return false;
        const int wgs = (N + c.bn - 1) / c.bn;
        const int nwk = c.threads / 64;
        int want = want_splits;
        if (want <= 0) {
            // aim for min(8, waves per workgroup) resident streaming waves per
            // CU, each with >= 2 stages
            const int waves = wgs * nwk;
            want = std::max(1, (kNumCUs * skinny_waves_per_cu(c)) / std::max(1, waves));
            want = std::min(want, std::max(1, stages_of(K) / (2 * nwk)));
        }
        split_stages(K, want, &pl.sps, &pl.splits);
        pl.grid = dim3(wgs, pl.splits, 1);
    } else {
        const int tm = (M + c.bm - 1) / c.bm, tn = (N + c.bn - 1) / c.bn;
        if (c.whole_k && (K % 512 != 0 || want_splits > 1)) return false;
        if (want_splits <= 0) {
            // the split count the cost model prefers (workspace below 2 GiB)
            bool have = false;
            Plan best{};
            for (int want : {1, 2, 4, 8}) {
                Plan cand;
                if (!make_plan(config, want, M, N, K, &cand)) continue;
                if (cand.ws_bytes >= (1ull << 31)) continue;
                if (!have || plan_cost(cand, M, N, K) < plan_cost(best, M, N, K)) {
                    best = cand;
                    have = true;
                }
            }
            if (have) *out = best;
            return have;
        }
        split_stages(K, want_splits, &pl.sps, &pl.splits);
        const int units = tm * tn * pl.splits;
        pl.grid = dim3(c.persistent ? std::min(units, kNumCUs * c.wgs_per_cu) : units, 1, 1);
    }
    pl.ws_bytes = pl.splits > 1 ? (size_t)pl.splits * M * N * 4 : 0;
    *out = pl;
    return true;
}

// Cost model: estimated time of a plan in ns, including the launch.
// Persistent kernels: rounds x (stages x stage time + per-unit time), where the
// stage time grows from cost.a (one workgroup per CU) to cost.b (wgs_per_cu
// of them); split-K adds the fp32 partial round trip (the reduce kernel).
// The constants were fitted to measured times (log-error least squares).
constexpr double kLaunchNs = 2000.0;
constexpr double kSplitBytesPerNs = 2084.0;
constexpr double kHbmBytesPerNs = 6000.0;
// A fragments re-read from L2 by every skinny workgroup (measured ~25 TB/s
// aggregate when they compete with the B stream).
constexpr double kL2BytesPerNs = 25000.0;

double plan_cost(const Plan& pl, int M, int N, int K)
{
    const Config& c = kConfigs[pl.config];
    const double split_ns =
        pl.splits > 1 ? (double)pl.splits * M * N * 4 * 2 / kSplitBytesPerNs + 1000.0 : 0.0;
    const double hbm_ns =
        ((double)M * K / 2 + (double)N * K / 2 + (double)(M + N) * K / 32 + 2.0 * M * N) /
        kHbmBytesPerNs;
    if (c.family == kSkinny) {
        // bandwidth-bound: needs skinny_waves_per_cu waves streaming B per CU
        const double wgs = (double)pl.grid.x * pl.grid.y;
        const double waves = wgs * (c.threads / 64);
        const double occ = std::min(1.0, waves / (kNumCUs * (double)skinny_waves_per_cu(c)));
        const double a_ns = (double)pl.grid.x * c.bm * (K / 2) / kL2BytesPerNs;
        return kLaunchNs + hbm_ns / (std::max(occ, 0.02) * c.cost.a) + a_ns + split_ns;
    }
    const double units = (double)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * pl.splits;
    const double slots = (double)kNumCUs * c.wgs_per_cu;
    const double rounds = std::ceil(units / slots);
    const double per_cu = std::ceil(std::min(units, slots) / kNumCUs);
    const double stage_us =
        c.wgs_per_cu == 1 ? c.cost.a
                          : c.cost.a + (c.cost.b - c.cost.a) * (per_cu - 1) / (c.wgs_per_cu - 1);
    const int stages = c.persistent ? (pl.sps + 3) / 4 * 4 : pl.sps;
    // Decode-sized M: a persistent kernel streams B only a few stages ahead and
    // leaves most MFMA rows empty; its HBM floor is taken at 60%.
    const double floor_ns = M <= 32 ? hbm_ns / 0.6 : hbm_ns;
    return kLaunchNs + std::max(rounds * (stages * stage_us + c.cost.c) * 1000.0, floor_ns) +
           split_ns;
}

// Measured best plans (graph-replayed timings of every configuration and
// split count on MI355X) for the shapes of the reference's published model
// layers, the BASELINE configurations and a few squares.  Exact matches
// take these; every other shape goes through the cost model.  Entries with
// "a / b us" were re-measured after the epilogue stores moved to LDS staging:
// medians of 7 interleaved rounds of the candidates, without / with MBS
// factors (a sweep run in order is biased by the clock's response to
// sustained load).  Entries naming an _m32 (32x32x64 MFMA) tile: medians of
// 3 x 7 interleaved rounds against the 16x16x128 tiles, without / with
// factors.  The five mid-M entries at K >= 5120 were re-measured (2 x 7
// rounds) after the 96-row tiles' A DMAs were dealt without fillers and the
// stage-top waits relaxed, which made the 96-row tiles 11-19% faster in
// all (their stage cost above is scaled by 0.87); six entries again after
// the pipelined epilogue (2 x 7 rounds; "before": not re-measured), and the
// three with fewer tiles than workgroup slots (1000, 3333 and 2048 x 2112
// rows) after their grids got the XCD remap.
struct TunedPlan {
    int M, N, K;
    const char* config;
    int splits;
};
const TunedPlan kTuned[] = {
    {1024, 17408, 5120, "bdirect_96x256_w1x4", 1},  // 51.48 / 55.27 us (96x256 m32: 53.20 / 57.22; 128x384 m32: 54.38 / 58.51)
    {1024, 1024, 5120, "bdirect_64x128_w1x2", 1},  // 10.7 us
    {256, 7168, 2048, "bdirect_64x128_w1x2", 1},  // 7.1 us
    {2048, 7168, 2048, "bdirect_256x256_w1x4", 1},  // 21.12 / 21.99 us (2x2: 21.59 / 22.76; 256x256 m32: 21.64 / 22.81)
    {256, 4096, 7168, "bdirect_64x128_w1x2", 1},  // 13.1 us
    {2048, 4096, 7168, "bdirect_128x256_w1x4_m32", 1},  // 32.17 / 33.43 us (128x256 1x4: 33.06 / 33.61; 96x256: 42.51 / 44.62 before)
    {256, 2112, 7168, "bdirect_64x128_w1x2", 2},  // 13.1 us
    {2048, 2112, 7168, "bdirect_96x256_w1x4_m32", 1},  // 22.76 / 23.57 us (96x256: 24.05 / 25.41)
    {1000, 1280, 512, "bdirect_64x128_w1x2", 1},  // 4.9 us
    {3333, 5120, 512, "bdirect_64x128_w1x2", 1},  // 15.3 us
    {1000, 5120, 12288, "bdirect_96x256_w1x4", 1},  // 36.67 / 37.82 us (96x256 m32: 37.12 / 38.05; 128x256 m32: 39.72 / 42.20)
    {3333, 1280, 12288, "bdirect_96x256_w1x4_m32", 1},  // 33.80 / 34.78 us (96x256: 35.83 / 36.99)
    {8192, 10240, 5120, "bdirect_256x256_w2x2", 1},  // 186.5 us
    {8192, 17408, 5120, "bdirect_192x256_w1x4", 1},  // 307.3 / 317.7 us (2x2: 313.1 / 320.9)
    {8192, 5120, 17408, "bdirect_256x256_w2x2", 1},  // 295.7 us
    {8192, 12288, 5120, "bdirect_256x256_w1x4", 1},  // 204.3 / 209.3 us (2x2: 205.4 / 211.6)
    {8192, 8192, 8192, "bdirect_256x256_w2x2", 1},  // 219.7 us
    {128, 256, 512, "bdirect_64x64_w1x1", 1},  // 4.5 us
    {4096, 4096, 4096, "bdirect_256x256_w2x2", 1},  // 35.3 us
    {512, 8192, 8192, "bdirect_64x256_w1x4", 1},  // 23.9 us
    {64, 8192, 8192, "bdirect_64x64_w1x1", 4},  // 13.5 us
    {2048, 2048, 2048, "bdirect_64x256_w1x4", 1},  // 9.4 us
};

int config_index(const char* name)
{
    for (int i = 0; i < kNumConfigs; ++i)
        if (std::strcmp(kConfigs[i].name, name) == 0) return i;
    return -1;
}

// skinny_only: choose among the decode (skinny) configurations only; for a
// shape whose unrestricted choice is skinny this is the same plan.
// max_bm: only configurations covering at most that many rows per tile.
bool choose_plan(int M, int N, int K, size_t ws_avail, Plan* best, bool skinny_only = false,
                 int max_bm = 1 << 30)
{
    for (const TunedPlan& t : kTuned) {
        if (t.M != M || t.N != N || t.K != K) continue;
        const int c = config_index(t.config);
        if (skinny_only && (c < 0 || kConfigs[c].family != kSkinny)) continue;
        if (c >= 0 && kConfigs[c].bm > max_bm) continue;
        Plan pl;
        if (c >= 0 && make_plan(c, t.splits, M, N, K, &pl) && pl.ws_bytes <= ws_avail) {
            *best = pl;
            return true;
        }
    }
    bool have = false;
    double best_cost = 0;
    for (int i = 0; i < kNumConfigs; ++i) {
        const bool skinny = kConfigs[i].family == kSkinny;
        if ((skinny_only && !skinny) || kConfigs[i].bm > max_bm) continue;
        for (int want : {0, 1, 2, 4, 8}) {
            if (skinny != (want == 0)) continue;  // skinny: its own split rule
            Plan pl;
            if (!make_plan(i, want, M, N, K, &pl)) continue;
            if (pl.ws_bytes > ws_avail || pl.ws_bytes >= (1ull << 31)) {
                if (!make_plan(i, 1, M, N, K, &pl)) continue;
            }
            const double cst = plan_cost(pl, M, N, K);
            if (!have || cst < best_cost) {
                *best = pl;
                best_cost = cst;
                have = true;
            }
        }
    }
    return have;
}

bool misaligned(const void* p, uintptr_t a) { return p && reinterpret_cast<uintptr_t>(p) % a != 0; }

int validate(const uint8_t* A, const uint8_t* B, const uint8_t* As, const uint8_t* Bs,
             const uint8_t* Af, const uint8_t* Bf, void* out, int M, int N, int K, int Mpad,
             int snp)
{
    // M == 0 (an empty batch) is valid: A, its scales, its factors and out
    // may then be the null data pointers of empty tensors.
    if (!B || !Bs || (M > 0 && (!A || !As || !out)))
        return fail(MBS_ERR_ARGUMENT, "null operand pointer");
    if ((Af == nullptr) != (Bf == nullptr) && M > 0)
        return fail(MBS_ERR_ARGUMENT, "AFactor and BFactor must be given together");
    // The kernels move A, B, the scales and the output in 16-byte units and
    // the factor bytes in dwords (buffer loads and LDS DMA at offsets that
    // are multiples of those sizes from each base).
    if (misaligned(A, 16) || misaligned(B, 16) || misaligned(As, 16) || misaligned(Bs, 16) ||
        misaligned(out, 16))
        return fail(MBS_ERR_ARGUMENT, "A, B, AScale, BScale and out must be 16-byte aligned");
    if (misaligned(Af, 4) || misaligned(Bf, 4))
        return fail(MBS_ERR_ARGUMENT, "AFactor and BFactor must be 4-byte aligned");
    if (M < 0 || N < 16 || K < 64)
        return fail(MBS_ERR_ARGUMENT, "need M >= 0, N >= 16, K >= 64; got M=" + std::to_string(M) +
                                          " N=" + std::to_string(N) + " K=" + std::to_string(K));
    if (N % 16) return fail(MBS_ERR_ARGUMENT, "N must be a multiple of 16, got " + std::to_string(N));
    if (K % 64)
        return fail(MBS_ERR_ARGUMENT, "K must be a multiple of 64 (16x16 B preshuffle), got " +
                                          std::to_string(K));
    if (Mpad != (M + 31) / 32 * 32)
        return fail(MBS_ERR_ARGUMENT, "Mpad must be round_up(M, 32)");
    if (snp != ((K + 31) / 32 + 7) / 8 * 8)
        return fail(MBS_ERR_ARGUMENT, "scaleN_pad must be round_up(ceil(K/32), 8)");
    // 32-bit buffer offsets: A and B are each one resource; the output and the
    // split-K workspace are addressed per tile (64-bit tile base, at most 256
    // rows below it), except in the decode kernel (M <= 32), which spans the
    // whole [M, N] output with one resource.
    if ((int64_t)512 * (K / 2) + 4096 >= (1ll << 31) || (int64_t)256 * N * 4 >= (1ll << 31) ||
        (int64_t)M * (K / 2) >= (1ll << 31) || (int64_t)N * (K / 2) >= (1ll << 31) ||
        (int64_t)std::min(M, 32) * N * 4 >= (1ll << 31))
        return fail(MBS_ERR_ARGUMENT, "problem too large for 32-bit buffer offsets");
    return MBS_OK;
}

// Arguments of the bf16-activation entry: x (bf16 [M, K]) takes the place
// of A and its scales; decode shapes only (M <= 8 with MBS factors).
int validate_from_bf16(const void* x, const uint8_t* B, const uint8_t* Bs, const uint8_t* Bf,
                       void* out, int M, int N, int K, int Mpad, int snp)
{
    if (M > 32)
        return fail(MBS_ERR_ARGUMENT, "the bf16-activation GEMM takes M <= 32 (decode shapes), got M=" +
                                          std::to_string(M));
    if (Bf && M > 8)
        return fail(MBS_ERR_ARGUMENT, "the bf16-activation GEMM with MBS factors takes M <= 8, got M=" +
                                          std::to_string(M));
    if (misaligned(Bf, 4)) return fail(MBS_ERR_ARGUMENT, "BFactor must be 4-byte aligned");
    if (M > 0 && !x) return fail(MBS_ERR_ARGUMENT, "null activation pointer");
    if (misaligned(x, 16)) return fail(MBS_ERR_ARGUMENT, "x must be 16-byte aligned");
    // The remaining checks are the packed entry's (x stands in for A and its
    // scale pointer; 32 rows of bf16 x stay below 2^31 bytes whenever the
    // K limit there holds).
    const uint8_t* xa = static_cast<const uint8_t*>(x);
    return validate(xa, B, xa, Bs, nullptr, nullptr, out, M, N, K, Mpad, snp);
}

// xbf: A is bf16 [M, K] quantized in registers (skinny plans only).
int run_plan(const Plan& pl, const uint8_t* A, const uint8_t* B, const uint8_t* As,
             const uint8_t* Bs, const uint8_t* Af, const uint8_t* Bf, void* out, int M, int N,
             int K, int snp, void* ws, size_t ws_bytes, void* stream, float alpha = 1.0f,
             const void* bias = nullptr, bool xbf = false)
{
    const Config& c = kConfigs[pl.config];
    if (xbf && !c.launch_xbf)
        return fail(MBS_ERR_CONFIG, std::string(c.name) + " has no bf16-activation variant");
    if (pl.ws_bytes > ws_bytes || (pl.ws_bytes && !ws))
        return fail(MBS_ERR_WORKSPACE, "workspace too small: need " + std::to_string(pl.ws_bytes) +
                                           " bytes");
    if (pl.ws_bytes && misaligned(ws, 16)) return fail(MBS_ERR_ARGUMENT, "workspace must be 16-byte aligned");
    if (misaligned(bias, 16)) return fail(MBS_ERR_ARGUMENT, "bias must be 16-byte aligned");
    GemmArgs a{};
    a.A = A; a.B = B; a.As = As; a.Bs = Bs; a.Af = Af; a.Bf = Bf;
    a.out = static_cast<uint16_t*>(out);
    a.ws = static_cast<float*>(ws);
    a.M = M; a.N = N; a.K = K; a.snp = snp;
    a.tiles_m = (M + c.bm - 1) / c.bm;
    a.tiles_n = (N + c.bn - 1) / c.bn;
    a.splits = pl.splits;
    a.sps = pl.sps;
    a.alpha = alpha;
    a.bias = static_cast<const uint16_t*>(bias);
    a.phase = g_phase;
    hipStream_t s = static_cast<hipStream_t>(stream);
    (void)hipGetLastError();  // do not report a stale error as ours
    // Persistent kernels take their general variant when a unit can have
    // dead stages (a split shorter than the others, or a stage count that is
    // not a multiple of 4) or K has a 64-wide tail; the others, their
    // constant-step variant.
    const int S_total = stages_of(K);
    const bool ktail = (K % 128) != 0;
    const bool gen = c.persistent ? (ktail || pl.sps % 4 != 0 || S_total % pl.sps != 0) : ktail;
    hipError_t e = (xbf ? c.launch_xbf : c.launch)(a, pl.grid, gen, pl.splits > 1, s);
    if (e != hipSuccess) return fail(MBS_ERR_LAUNCH, std::string("launch failed: ") + hipGetErrorString(e));
    if (pl.splits > 1) {
        const int64_t quads = (int64_t)M * (N / 4);
        dim3 g((unsigned)((quads + 255) / 256));
        hipLaunchKernelGGL(splitk_reduce_kernel, g, dim3(256), 0, s, a);
        e = hipGetLastError();
        if (e != hipSuccess)
            return fail(MBS_ERR_LAUNCH, std::string("reduce launch failed: ") + hipGetErrorString(e));
    }
    return MBS_OK;
}

// ------------------------------------------------------------ grouped GEMM
// Persistent configurations with a grouped (MoE) variant; `dense` names the
// dense configuration whose cost constants rank them.
struct GroupedConfig {
    const char* dense;
    hipError_t (*launch)(const GemmArgs&, dim3, bool, bool, hipStream_t);
};
const GroupedConfig kGrouped[] = {
    {"bdirect_256x256_w2x2", launch_bdirect_grouped<B256x256>},
    {"bdirect_128x256_w1x4", launch_bdirect_grouped<B128x256w14>},
    {"bdirect_64x256_w1x4", launch_bdirect_grouped<B64x256>},
    {"bdirect_64x128_w1x2", launch_bdirect_grouped<B64x128>},
    // 32x32x64-MFMA tiles: whole-K plans only (K % 512 == 0)
    {"bdirect_128x256_w1x4_m32", launch_bdirect_grouped<B128x256m>},
    {"bdirect_256x256_w1x4_m32", launch_bdirect_grouped<B256x256m>},
};
constexpr int kNumGrouped = (int)(sizeof(kGrouped) / sizeof(kGrouped[0]));

// Upper bound of the grouped tile count: every expert adds at most one
// partial M-tile to the ceil(M / BM) full ones.
int grouped_units_bound(const Config& c, int M, int N, int E)
{
    return ((M + c.bm - 1) / c.bm + E) * ((N + c.bn - 1) / c.bn);
}

// Config choice: the dense cost model at the tile count the experts' padded
// row blocks give on average (half a tile of padding per expert).
// Measured best grouped configurations (graph-replayed, every configuration)
// for configs[3]'s expert shapes at 8 experts x 256 tokens; exact matches on
// (M, N, K, E) take these, everything else goes through the cost model.
struct TunedGrouped {
    int M, N, K, E;
    const char* dense;
};
const TunedGrouped kTunedGrouped[] = {
    // medians of 7 interleaved rounds of every configuration (us): chosen / others
    {2048, 7168, 2048, 8, "bdirect_256x256_w1x4_m32"},  // 24.8 / 256x256 2x2 25.4, 128x256 26.1, m32 128x256 27.6
    {2048, 4096, 7168, 8, "bdirect_128x256_w1x4"},  // 34.3 / 64x256 39.1, m32 128x256 39.3, m32 256x256 44.5
    {2048, 2112, 7168, 8, "bdirect_128x256_w1x4_m32"},  // 26.2 / 128x256 27.1, 64x128 29.6, 64x256 33.5
};

int choose_grouped(int M, int N, int K, int E)
{
    for (const TunedGrouped& t : kTunedGrouped) {
        if (t.M != M || t.N != N || t.K != K || t.E != E) continue;
        for (int g = 0; g < kNumGrouped; ++g)
            if (std::strcmp(kGrouped[g].dense, t.dense) == 0) return g;
    }
    int best = 0;
    double best_cost = 0;
    for (int g = 0; g < kNumGrouped; ++g) {
        const int c = config_index(kGrouped[g].dense);
        const int Meff = M + E * kConfigs[c].bm / 2;
        Plan pl;
        if (!make_plan(c, 1, Meff, N, K, &pl)) continue;
        const double cst = plan_cost(pl, Meff, N, K);
        if (g == 0 || cst < best_cost) {
            best = g;
            best_cost = cst;
        }
    }
    return best;
}

int run_grouped(int g, const uint8_t* A, const uint8_t* B, const uint8_t* As, const uint8_t* Bs,
                const uint8_t* Af, const uint8_t* Bf, const int* groups, int E, void* out, int M,
                int N, int K, int snp, void* stream, float alpha, const void* bias)
{
    const Config& c = kConfigs[config_index(kGrouped[g].dense)];
    if (c.whole_k && K % 512 != 0)
        return fail(MBS_ERR_CONFIG, std::string(c.name) + " cannot run K=" + std::to_string(K) +
                                        " (whole-K tiles need K % 512 == 0)");
    GemmArgs a{};
    a.A = A; a.B = B; a.As = As; a.Bs = Bs; a.Af = Af; a.Bf = Bf;
    a.out = static_cast<uint16_t*>(out);
    a.M = M; a.N = N; a.K = K; a.snp = snp;
    a.tiles_m = 0;  // computed on the device from the expert offsets
    a.tiles_n = (N + c.bn - 1) / c.bn;
    split_stages(K, 1, &a.sps, &a.splits);
    a.groups = groups;
    a.n_groups = E;
    a.alpha = alpha;
    a.bias = static_cast<const uint16_t*>(bias);
    a.phase = g_phase;
    const int S_total = stages_of(K);
    const bool gen = (K % 128) != 0 || a.sps % 4 != 0 || S_total % a.sps != 0;
    const int units = grouped_units_bound(c, M, N, E);
    const dim3 grid((unsigned)std::min(units, kNumCUs * c.wgs_per_cu));
    (void)hipGetLastError();
    const hipError_t e = kGrouped[g].launch(a, grid, gen, false, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(MBS_ERR_LAUNCH, std::string("launch failed: ") + hipGetErrorString(e));
    return MBS_OK;
}

// Device address of `scratch` on the current device, looked up once per
// device (nullptr if the lookup fails; the error text is recorded).
constexpr int kMaxDevices = 64;
void* scratch_on_current_device()
{
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_last_error("no current HIP device for the scratch buffer");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_last_error((std::string("hipGetSymbolAddress(scratch) failed: ") +
                            hipGetErrorString(e)).c_str());
            return nullptr;
        }
        addr[dev] = ptr;
    }
    return addr[dev];
}

}  // namespace
}  // namespace mbs

using namespace mbs;

extern "C" {

const char* mbs_status_string(int status)
{
    switch (status) {
    case MBS_OK: return "ok";
    case MBS_ERR_ARGUMENT: return "invalid argument";
    case MBS_ERR_WORKSPACE: return "workspace too small";
    case MBS_ERR_LAUNCH: return "kernel launch failed";
    case MBS_ERR_CONFIG: return "invalid kernel configuration";
    default: return "unknown status";
    }
}

const char* mbs_last_error(void) { return g_last_error.c_str(); }

size_t mbs_gemm_a4w4_workspace_bytes(int M, int N, int K)
{
    if (M < 1 || N < 16 || K < 64 || N % 16 || K % 64) return 0;
    Plan pl;
    if (!choose_plan(M, N, K, (size_t)1 << 31, &pl)) return 0;
    return pl.ws_bytes;
}

int mbs_gemm_a4w4_launch(const uint8_t* A, const uint8_t* B, const uint8_t* AScale,
                         const uint8_t* BScale, const uint8_t* AFactor, const uint8_t* BFactor,
                         void* out, int M, int N, int K, int Mpad, int scaleN_pad,
                         void* workspace, size_t workspace_bytes, void* stream)
{
    set_last_error("");
    int st = validate(A, B, AScale, BScale, AFactor, BFactor, out, M, N, K, Mpad, scaleN_pad);
    if (st != MBS_OK || M == 0) return st;
    Plan pl;
    if (!choose_plan(M, N, K, workspace ? workspace_bytes : 0, &pl))
        return fail(MBS_ERR_CONFIG, "no kernel configuration fits this problem");
    return run_plan(pl, A, B, AScale, BScale, AFactor, BFactor, out, M, N, K, scaleN_pad,
                    workspace, workspace_bytes, stream);
}

int mbs_gemm_a4w4_grouped_launch(const uint8_t* A, const uint8_t* B, const uint8_t* AScale,
                                 const uint8_t* BScale, const uint8_t* AFactor,
                                 const uint8_t* BFactor, const int* group_offsets, int num_groups,
                                 void* out, int M, int N, int K, int Mpad, int scaleN_pad,
                                 int config, void* stream)
{
    return mbs_gemm_a4w4_grouped_launch_ex(A, B, AScale, BScale, AFactor, BFactor, group_offsets,
                                           num_groups, out, M, N, K, Mpad, scaleN_pad, 1.0f, nullptr,
                                           config, stream);
}

int mbs_gemm_a4w4_grouped_launch_ex(const uint8_t* A, const uint8_t* B, const uint8_t* AScale,
                                    const uint8_t* BScale, const uint8_t* AFactor,
                                    const uint8_t* BFactor, const int* group_offsets,
                                    int num_groups, void* out, int M, int N, int K, int Mpad,
                                    int scaleN_pad, float alpha, const void* bias, int config,
                                    void* stream)
{
    set_last_error("");
    int st = validate(A, B, AScale, BScale, AFactor, BFactor, out, M, N, K, Mpad, scaleN_pad);
    if (st != MBS_OK) return st;
    if (!group_offsets) return fail(MBS_ERR_ARGUMENT, "null group_offsets");
    if (num_groups < 1 || num_groups > kMaxGroups)
        return fail(MBS_ERR_ARGUMENT, "num_groups must be in [1, " + std::to_string(kMaxGroups) + "]");
    const int64_t Npad = (N + 31) / 32 * 32;
    if ((int64_t)num_groups * N * (K / 2) >= (1ll << 31) ||
        (int64_t)num_groups * Npad * scaleN_pad >= (1ll << 31) || (int64_t)num_groups * N >= (1ll << 31))
        return fail(MBS_ERR_ARGUMENT, "stacked expert weights too large for 32-bit buffer offsets");
    if (config < -1 || config >= kNumGrouped)
        return fail(MBS_ERR_CONFIG, "grouped config out of range");
    if (!(alpha == alpha)) return fail(MBS_ERR_ARGUMENT, "alpha is NaN");
    if (misaligned(group_offsets, 4)) return fail(MBS_ERR_ARGUMENT, "group_offsets must be 4-byte aligned");
    if (misaligned(bias, 16)) return fail(MBS_ERR_ARGUMENT, "bias must be 16-byte aligned");
    if (M == 0) return MBS_OK;
    const int g = config >= 0 ? config : choose_grouped(M, N, K, num_groups);
    return run_grouped(g, A, B, AScale, BScale, AFactor, BFactor, group_offsets, num_groups, out, M,
                       N, K, scaleN_pad, stream, alpha, bias);
}

int mbs_gemm_a4w4_check_groups(const int* group_offsets, int num_groups, int M, uint32_t* status,
                               void* stream)
{
    set_last_error("");
    if (!group_offsets || !status) return fail(MBS_ERR_ARGUMENT, "null group_offsets or status");
    if (num_groups < 1 || num_groups > kMaxGroups)
        return fail(MBS_ERR_ARGUMENT, "num_groups must be in [1, " + std::to_string(kMaxGroups) + "]");
    if (M < 0) return fail(MBS_ERR_ARGUMENT, "M must be >= 0");
    if (reinterpret_cast<uintptr_t>(group_offsets) % 4 || reinterpret_cast<uintptr_t>(status) % 4)
        return fail(MBS_ERR_ARGUMENT, "group_offsets and status must be 4-byte aligned");
    (void)hipGetLastError();
    hipLaunchKernelGGL(check_groups_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream),
                       group_offsets, num_groups, M, status);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MBS_ERR_LAUNCH, std::string("launch failed: ") + hipGetErrorString(e));
    return MBS_OK;
}

int mbs_gemm_a4w4_grouped_num_configs(void) { return kNumGrouped; }

const char* mbs_gemm_a4w4_grouped_config_name(int config)
{
    return (config >= 0 && config < kNumGrouped) ? kGrouped[config].dense : "";
}

int mbs_gemm_a4w4_num_configs(void) { return kNumConfigs; }

const char* mbs_gemm_a4w4_config_name(int config)
{
    return (config >= 0 && config < kNumConfigs) ? kConfigs[config].name : "";
}

int mbs_gemm_a4w4_plan_name(int M, int N, int K, char* buf, size_t buf_len)
{
    Plan pl;
    if (M < 1 || N < 16 || K < 64 || N % 16 || K % 64 || !choose_plan(M, N, K, (size_t)1 << 31, &pl))
        return MBS_ERR_ARGUMENT;
    if (buf && buf_len)
        snprintf(buf, buf_len, "%s splits=%d grid=%ux%u ws=%zu", kConfigs[pl.config].name,
                 pl.splits, pl.grid.x, pl.grid.y, pl.ws_bytes);
    return MBS_OK;
}

size_t mbs_gemm_a4w4_config_workspace_bytes(int config, int splits, int M, int N, int K)
{
    Plan pl;
    if (!make_plan(config, splits, M, N, K, &pl)) return 0;
    return pl.ws_bytes;
}

int mbs_gemm_a4w4_launch_config(int config, int splits, const uint8_t* A, const uint8_t* B,
                                const uint8_t* AScale, const uint8_t* BScale,
                                const uint8_t* AFactor, const uint8_t* BFactor, void* out, int M,
                                int N, int K, int Mpad, int scaleN_pad, void* workspace,
                                size_t workspace_bytes, void* stream)
{
    set_last_error("");
    int st = validate(A, B, AScale, BScale, AFactor, BFactor, out, M, N, K, Mpad, scaleN_pad);
    if (st != MBS_OK) return st;
    if (config < 0 || config >= kNumConfigs)
        return fail(MBS_ERR_CONFIG, "config " + std::to_string(config) + " out of range");
    if (M == 0) return MBS_OK;
    Plan pl;
    if (!make_plan(config, splits, M, N, K, &pl))
        return fail(MBS_ERR_CONFIG, "config " + std::to_string(config) + " cannot run M=" +
                                        std::to_string(M) + " K=" + std::to_string(K) + " with " +
                                        std::to_string(splits) + " splits");
    return run_plan(pl, A, B, AScale, BScale, AFactor, BFactor, out, M, N, K, scaleN_pad,
                    workspace, workspace_bytes, stream);
}

int mbs_gemm_a4w4_launch_ex(int config, int splits, const uint8_t* A, const uint8_t* B,
                            const uint8_t* AScale, const uint8_t* BScale, const uint8_t* AFactor,
                            const uint8_t* BFactor, void* out, int M, int N, int K, int Mpad,
                            int scaleN_pad, float alpha, const void* bias, void* workspace,
                            size_t workspace_bytes, void* stream)
{
    set_last_error("");
    int st = validate(A, B, AScale, BScale, AFactor, BFactor, out, M, N, K, Mpad, scaleN_pad);
    if (st != MBS_OK) return st;
    if (!(alpha == alpha)) return fail(MBS_ERR_ARGUMENT, "alpha is NaN");
    if (config >= kNumConfigs)
        return fail(MBS_ERR_CONFIG, "config " + std::to_string(config) + " out of range");
    if (M == 0) return MBS_OK;
    Plan pl;
    if (config < 0) {
        if (!choose_plan(M, N, K, workspace ? workspace_bytes : 0, &pl))
            return fail(MBS_ERR_CONFIG, "no kernel configuration fits this problem");
    } else if (!make_plan(config, splits, M, N, K, &pl)) {
        return fail(MBS_ERR_CONFIG, "config " + std::to_string(config) + " cannot run M=" +
                                        std::to_string(M) + " K=" + std::to_string(K) + " with " +
                                        std::to_string(splits) + " splits");
    }
    return run_plan(pl, A, B, AScale, BScale, AFactor, BFactor, out, M, N, K, scaleN_pad,
                    workspace, workspace_bytes, stream, alpha, bias);
}

size_t mbs_gemm_a4w4_from_bf16_workspace_bytes(int M, int N, int K)
{
    if (M < 1 || M > 32 || N < 16 || K < 64 || N % 16 || K % 64) return 0;
    Plan pl;
    if (!choose_plan(M, N, K, (size_t)1 << 31, &pl, true)) return 0;
    return pl.ws_bytes;
}

int mbs_gemm_a4w4_from_bf16_launch(int config, int splits, const void* x, const uint8_t* B,
                                   const uint8_t* BScale, const uint8_t* BFactor, void* out, int M,
                                   int N, int K, int Mpad, int scaleN_pad, float alpha,
                                   const void* bias, void* workspace, size_t workspace_bytes,
                                   void* stream)
{
    set_last_error("");
    int st = validate_from_bf16(x, B, BScale, BFactor, out, M, N, K, Mpad, scaleN_pad);
    if (st != MBS_OK) return st;
    if (!(alpha == alpha)) return fail(MBS_ERR_ARGUMENT, "alpha is NaN");
    if (config >= kNumConfigs || (config >= 0 && kConfigs[config].family != kSkinny))
        return fail(MBS_ERR_CONFIG, "config " + std::to_string(config) +
                                        " is not a decode (skinny) configuration");
    // MBS: one 16-row tile (the compact forms) and no K split, since every
    // workgroup derives the row factors from the whole row
    const bool mbs = BFactor != nullptr;
    if (mbs && config >= 0 && (kConfigs[config].bm != 16 || splits > 1))
        return fail(MBS_ERR_CONFIG, "with MBS factors the config must be a 16-row decode "
                                    "configuration without K splits");
    if (M == 0) return MBS_OK;
    Plan pl;
    if (config < 0) {
        if (!choose_plan(M, N, K, mbs ? 0 : (workspace ? workspace_bytes : 0), &pl, true,
                         mbs ? 16 : 1 << 30))
            return fail(MBS_ERR_CONFIG, "no decode configuration fits this problem");
    } else if (!make_plan(config, mbs ? 1 : splits, M, N, K, &pl)) {
        return fail(MBS_ERR_CONFIG, "config " + std::to_string(config) + " cannot run M=" +
                                        std::to_string(M) + " K=" + std::to_string(K) + " with " +
                                        std::to_string(splits) + " splits");
    }
    return run_plan(pl, static_cast<const uint8_t*>(x), B, nullptr, BScale, nullptr, BFactor, out,
                    M, N, K, scaleN_pad, workspace, workspace_bytes, stream, alpha, bias, true);
}

#if MBS_PHASE_TIMER
// Timer builds (libmbs_gemm_phase.so) only: every later persistent-kernel
// launch adds its phase sums into `sums` (kPhSlots device words per
// workgroup, 1024 workgroups at most, cleared by
// the caller); nullptr detaches.
void mbs_phase_timer_attach(unsigned long long* sums) { g_phase = sums; }
int mbs_phase_timer_slots(void) { return kPhSlots; }
#endif

int mbs_gemm_a4w4_launch_noalloc(int config, int splits, const uint8_t* A, const uint8_t* B,
                                 const uint8_t* AScale, const uint8_t* BScale,
                                 const uint8_t* AFactor, const uint8_t* BFactor, void* out, int M,
                                 int N, int K, int Mpad, int scaleN_pad, float alpha,
                                 const void* bias, void* stream)
{
    set_last_error("");
    int st = validate(A, B, AScale, BScale, AFactor, BFactor, out, M, N, K, Mpad, scaleN_pad);
    if (st != MBS_OK) return st;
    if (!(alpha == alpha)) return fail(MBS_ERR_ARGUMENT, "alpha is NaN");
    if (config >= kNumConfigs)
        return fail(MBS_ERR_CONFIG, "config " + std::to_string(config) + " out of range");
    if (M == 0) return MBS_OK;
    const size_t cap = MBS_NOALLOC_SCRATCH_BYTES;
    Plan pl;
    if (config < 0) {
        // the heuristic, limited to plans whose partials fit the scratch
        if (!choose_plan(M, N, K, cap, &pl))
            return fail(MBS_ERR_CONFIG, "no kernel configuration fits this problem");
    } else {
        if (!make_plan(config, splits, M, N, K, &pl))
            return fail(MBS_ERR_CONFIG, "config " + std::to_string(config) + " cannot run M=" +
                                            std::to_string(M) + " K=" + std::to_string(K) + " with " +
                                            std::to_string(splits) + " splits");
        // the config's own split choice falls back to no split when its
        // partials do not fit; an explicit split count is refused
        if (pl.ws_bytes > cap && splits <= 0 && !make_plan(config, 1, M, N, K, &pl))
            return fail(MBS_ERR_CONFIG, "config " + std::to_string(config) + " cannot run M=" +
                                            std::to_string(M) + " K=" + std::to_string(K) + " with " +
                                            std::to_string(splits) + " splits");
    }
    if (pl.ws_bytes > cap)
        return fail(MBS_ERR_WORKSPACE, "split-K partials need " + std::to_string(pl.ws_bytes) +
                                           " bytes; the allocation-free entry point has " +
                                           std::to_string(cap) + " bytes of scratch");
    void* ws = nullptr;
    if (pl.ws_bytes) {
        ws = scratch_on_current_device();
        if (!ws) return MBS_ERR_LAUNCH;
    }
    return run_plan(pl, A, B, AScale, BScale, AFactor, BFactor, out, M, N, K, scaleN_pad, ws,
                    pl.ws_bytes, stream, alpha, bias);
}

}  // extern "C"
