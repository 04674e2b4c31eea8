// Launchers, buffers, weight upload and the device transformer block.
#include "runtime.hpp"

#include <math.h>
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "attention.hpp"
#include "attention_bf16.hpp"
#include "attention_split.hpp"
#include "attention_h2.hpp"
#include "band_attention.hpp"
#include "elementwise.hpp"
#include "gemm.hpp"
#include "gemm_bf16.hpp"
#include "gemm_split.hpp"
#include "gemm_h2.hpp"

namespace vh {

// ----------------------------------------------------------------- errors
static std::mutex g_err_mu;
static char g_err[1024] = "";

void set_error(const char *fmt, ...) {
    std::lock_guard<std::mutex> lock(g_err_mu);
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

const char *last_error() { return g_err; }

bool check(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    set_error("%s failed: %s", what, hipGetErrorString(e));
    return false;
}

bool debug_enabled() {
    static int on = -1;
    if (on < 0) on = getenv("VOCALARC_GPU_DEBUG") != nullptr;
    return on != 0;
}

// After each launch: pick up launch errors; in debug mode synchronise and log
// (native/native_gpu_cuda.cu:487-495 offers the same switch).
bool sync_debug(hipStream_t s, const char *what) {
    if (!check(hipGetLastError(), what)) return false;
    if (!debug_enabled()) return true;
    bool ok = check(hipStreamSynchronize(s), what);
    fprintf(stderr, "vocalarc-hip: %s %s\n", what, ok ? "ok" : last_error());
    return ok;
}

// ---------------------------------------------------------------- buffers
bool DeviceBuffer::ensure(size_t need, const char *what) {
    if (need <= bytes && ptr != nullptr) return true;
    release();
    if (need == 0) need = 16;
    if (!check(hipMalloc(&ptr, need), what)) {
        ptr = nullptr;
        return false;
    }
    bytes = need;
    return true;
}

void DeviceBuffer::release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
}

// ----------------------------------------------------------------- timing
bool KernelTimer::wants(const char *name) const {
    if (all) return true;
    for (const auto &n : only)
        if (n == name) return true;
    return false;
}

void KernelTimer::begin(hipStream_t s, const char *, hipEvent_t *a) {
    (void)hipEventCreate(a);
    (void)hipEventRecord(*a, s);
}

void KernelTimer::end(hipStream_t s, const char *name, hipEvent_t a) {
    hipEvent_t b;
    (void)hipEventCreate(&b);
    (void)hipEventRecord(b, s);
    pending.push_back({name, a, b});
}

void KernelTimer::collect() {
    for (auto &p : pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(p.b) == hipSuccess && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            auto &t = totals[p.name];
            t.first += ms;
            t.second += 1;
        }
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    pending.clear();
}

void KernelTimer::reset() {
    collect();
    totals.clear();
}

// --------------------------------------------------------------- launchers
static inline unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

// Output columns a GEMM writes per row (GELU-GLU halves them).
static int out_cols(int N, int epilogue) { return epilogue == EPI_GEGLU ? N / 2 : N; }

static bool gemm_ok(const GemmArgs &g) {
    if (g.M <= 0 || g.N <= 0 || g.K <= 0) return false;
    if (g.K % 4 || g.lda % 4 || g.ldb % 4 || g.lda < g.K || g.ldb < g.K) return false;
    if (((uintptr_t)g.A | (uintptr_t)g.B) & 15) return false;
    if (g.M > INT32_MAX / 2) return false;
    return true;
}

template <int EPI>
static void launch_epi(hipStream_t s, const GemmDesc *single, const GemmBatch *batch, unsigned tiles, unsigned n) {
    if (single) hipLaunchKernelGGL(gemm_f32_kernel<EPI>, dim3(tiles), dim3(GEMM_THREADS), 0, s, *single);
    else hipLaunchKernelGGL(gemm_f32_batched_kernel<EPI>, dim3(tiles, 1, n), dim3(GEMM_THREADS), 0, s, *batch);
}

static bool launch_gemm(hipStream_t s, int epi, const GemmDesc *single, const GemmBatch *batch, unsigned tiles,
                        unsigned n) {
    switch (epi) {
        case EPI_STORE: launch_epi<EPI_STORE>(s, single, batch, tiles, n); break;
        case EPI_GELU: launch_epi<EPI_GELU>(s, single, batch, tiles, n); break;
        case EPI_TANH: launch_epi<EPI_TANH>(s, single, batch, tiles, n); break;
        case EPI_RESIDUAL: launch_epi<EPI_RESIDUAL>(s, single, batch, tiles, n); break;
        case EPI_GEGLU: launch_epi<EPI_GEGLU>(s, single, batch, tiles, n); break;
        default: set_error("unknown GEMM epilogue %d", epi); return false;
    }
    return sync_debug(s, "gemm_f32_kernel");
}

static GemmDesc to_desc(const GemmArgs &g) {
    GemmDesc d;
    d.A = g.A; d.B = g.B; d.bias = g.bias; d.C = g.C;
    d.M = (int)g.M; d.N = g.N; d.K = g.K;
    d.lda = g.lda; d.ldb = g.ldb; d.ldc = g.ldc;
    return d;
}

static int64_t tiles_of(const GemmArgs &g) {
    return ((g.M + GEMM_BM - 1) / GEMM_BM) * ((g.N + GEMM_BN - 1) / GEMM_BN);
}

bool gemm(hipStream_t s, const GemmArgs &g, int epilogue, KernelTimer *t, const char *name) {
    if (!gemm_ok(g) || g.ldc < out_cols(g.N, epilogue)) {
        set_error("gemm: unsupported shape M=%lld N=%d K=%d lda=%d ldb=%d", (long long)g.M, g.N, g.K, g.lda, g.ldb);
        return false;
    }
    if (epilogue == EPI_GEGLU && g.N % 64) {
        set_error("gemm: GELU-GLU needs N %% 64 == 0 (N=%d)", g.N);
        return false;
    }
    GemmDesc d = to_desc(g);
    Scope sc(t, s, name);
    return launch_gemm(s, epilogue, &d, nullptr, (unsigned)tiles_of(g), 1);
}

bool gemm_batched(hipStream_t s, const std::vector<GemmArgs> &gs, int epilogue, KernelTimer *t, const char *name) {
    Scope sc(t, s, name);
    for (size_t first = 0; first < gs.size(); first += GEMM_MAX_BATCH) {
        const size_t count = std::min(gs.size() - first, (size_t)GEMM_MAX_BATCH);
        GemmBatch b;
        memset(&b, 0, sizeof(b));
        int64_t max_tiles = 0;
        for (size_t i = 0; i < count; i++) {
            const GemmArgs &g = gs[first + i];
            if (!gemm_ok(g) || g.ldc < out_cols(g.N, epilogue) || (epilogue == EPI_GEGLU && g.N % 64)) {
                set_error("gemm_batched: unsupported shape M=%lld N=%d K=%d", (long long)g.M, g.N, g.K);
                return false;
            }
            b.d[i] = to_desc(g);
            max_tiles = std::max(max_tiles, tiles_of(g));
        }
        if (!launch_gemm(s, epilogue, nullptr, &b, (unsigned)max_tiles, (unsigned)count)) return false;
    }
    return true;
}

// ------------------------------------------------------------ bf16 GEMM
static bool gemm_bf16_ok(const GemmArgsBF16 &g, int epilogue) {
    if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.M > INT32_MAX / 2) return false;
    if (g.K % 4 || g.lda % 4 || g.lda < g.K || g.ldb % 8 || g.ldb < bf16_pitch(g.K)) return false;
    if (g.a_bf16 && (g.K % 8 || g.lda % 8)) return false;
    // the epilogue's row offsets within a wave's rows are 32-bit
    if (g.ldc < out_cols(g.N, epilogue) || g.ldc > (1 << 21) || (epilogue == EPI_GEGLU && g.N % 64)) return false;
    if (g.c_bf16 && epilogue == EPI_RESIDUAL) return false;
    if (((uintptr_t)g.A | (uintptr_t)g.B) & 15) return false;
    return true;
}

static GemmDescBF16 to_desc_bf16(const GemmArgsBF16 &g) {
    GemmDescBF16 d;
    d.A = g.A; d.B = static_cast<const bf16 *>(g.B); d.bias = g.bias; d.C = g.C;
    d.M = (int)g.M; d.N = g.N; d.K = g.K;
    d.lda = g.lda; d.ldb = g.ldb; d.ldc = g.ldc;
    return d;
}

// bf16 GEMM tiling: 8 waves in a 4 x 2 grid, 2 x 2 accumulators (64 x 64) per
// wave, a 256 x 128 block, K chunks of 32; two workgroups per CU (60 KB of LDS
// each) = 4 waves per SIMD (122 VGPRs).  With bf16 A and K % 32 == 0 the same
// block runs as the global->LDS DMA ring (gemm_bf16_dma_kernel: 72 KB of LDS,
// two workgroups per CU), which keeps twice the bytes in flight.
constexpr int BF_WM = 4, BF_WN = 2, BF_FM = 2, BF_FN = 2, BF_BK = 32, BF_OCC = 2;
using BFTile = BF16Tile<BF_WM, BF_WN, BF_FM, BF_FN>;
static_assert(BFTile::BM == GBD_BM && BFTile::BN == GBD_BN && BFTile::THREADS == GBD_THREADS,
              "the DMA ring runs the register-staged kernel's block");

static int64_t tiles_bf16(const GemmArgsBF16 &g) {
    return ((g.M + BFTile::BM - 1) / BFTile::BM) * ((g.N + BFTile::BN - 1) / BFTile::BN);
}

// The DMA ring takes whole 32-element K chunks of bf16 A (16-byte aligned
// rows, which gemm_bf16_ok already requires of bf16 A) and row pitches whose
// 256-row offsets fit its 32-bit lane offsets.
static bool dma_ok(const GemmArgsBF16 &g) {
    return g.a_bf16 && g.K % GBD_BK == 0 && !g.staged && g.lda <= (1 << 21) && g.ldb <= (1 << 21);
}

template <int EPI, typename TA, typename TC>
static void launch_bf16_typed(hipStream_t s, const GemmDescBF16 *single, const GemmBatchBF16 *batch, unsigned tiles,
                              unsigned n, bool dma) {
    if constexpr (std::is_same<TA, bf16>::value) {
        if (dma) {
            if (single)
                hipLaunchKernelGGL((gemm_bf16_dma_kernel<EPI, TC>), dim3(tiles), dim3(GBD_THREADS), 0, s, *single);
            else
                hipLaunchKernelGGL((gemm_bf16_dma_batched_kernel<EPI, TC>), dim3(tiles, 1, n), dim3(GBD_THREADS), 0,
                                   s, *batch);
            return;
        }
    }
    if (single)
        hipLaunchKernelGGL((gemm_bf16_kernel<EPI, TA, TC, BF_BK, BF_WM, BF_WN, BF_FM, BF_FN, BF_OCC>), dim3(tiles),
                           dim3(BFTile::THREADS), 0, s, *single);
    else
        hipLaunchKernelGGL((gemm_bf16_batched_kernel<EPI, TA, TC, BF_BK, BF_WM, BF_WN, BF_FM, BF_FN, BF_OCC>),
                           dim3(tiles, 1, n), dim3(BFTile::THREADS), 0, s, *batch);
}

template <int EPI>
static void launch_bf16_epi(hipStream_t s, bool a16, bool c16, const GemmDescBF16 *single, const GemmBatchBF16 *batch,
                            unsigned tiles, unsigned n, bool dma) {
    if constexpr (EPI == EPI_RESIDUAL) {
        if (a16) launch_bf16_typed<EPI, bf16, float>(s, single, batch, tiles, n, dma);
        else launch_bf16_typed<EPI, float, float>(s, single, batch, tiles, n, dma);
    } else {
        if (a16 && c16) launch_bf16_typed<EPI, bf16, bf16>(s, single, batch, tiles, n, dma);
        else if (a16) launch_bf16_typed<EPI, bf16, float>(s, single, batch, tiles, n, dma);
        else if (c16) launch_bf16_typed<EPI, float, bf16>(s, single, batch, tiles, n, dma);
        else launch_bf16_typed<EPI, float, float>(s, single, batch, tiles, n, dma);
    }
}

static bool launch_bf16(hipStream_t s, int epi, bool a16, bool c16, const GemmDescBF16 *single,
                        const GemmBatchBF16 *batch, unsigned tiles, unsigned n, bool dma) {
    switch (epi) {
        case EPI_STORE: launch_bf16_epi<EPI_STORE>(s, a16, c16, single, batch, tiles, n, dma); break;
        case EPI_GELU: launch_bf16_epi<EPI_GELU>(s, a16, c16, single, batch, tiles, n, dma); break;
        case EPI_TANH: launch_bf16_epi<EPI_TANH>(s, a16, c16, single, batch, tiles, n, dma); break;
        case EPI_RESIDUAL: launch_bf16_epi<EPI_RESIDUAL>(s, a16, c16, single, batch, tiles, n, dma); break;
        case EPI_GEGLU: launch_bf16_epi<EPI_GEGLU>(s, a16, c16, single, batch, tiles, n, dma); break;
        default: set_error("unknown GEMM epilogue %d", epi); return false;
    }
    return sync_debug(s, dma ? "gemm_bf16_dma_kernel" : "gemm_bf16_kernel");
}

bool gemm_bf16(hipStream_t s, const GemmArgsBF16 &g, int epilogue, KernelTimer *t, const char *name) {
    if (!gemm_bf16_ok(g, epilogue)) {
        set_error("gemm_bf16: unsupported shape M=%lld N=%d K=%d lda=%d ldb=%d", (long long)g.M, g.N, g.K, g.lda,
                  g.ldb);
        return false;
    }
    GemmDescBF16 d = to_desc_bf16(g);
    Scope sc(t, s, name);
    return launch_bf16(s, epilogue, g.a_bf16, g.c_bf16, &d, nullptr, (unsigned)tiles_bf16(g), 1,
                       dma_ok(g));
}

bool gemm_bf16_batched(hipStream_t s, const std::vector<GemmArgsBF16> &gs, int epilogue, KernelTimer *t,
                       const char *name) {
    Scope sc(t, s, name);
    for (size_t first = 0; first < gs.size(); first += GB_MAX_BATCH) {
        const size_t count = std::min(gs.size() - first, (size_t)GB_MAX_BATCH);
        GemmBatchBF16 b;
        memset(&b, 0, sizeof(b));
        int64_t max_tiles = 0;
        bool dma = true;
        for (size_t i = 0; i < count; i++) {
            const GemmArgsBF16 &g = gs[first + i];
            if (!gemm_bf16_ok(g, epilogue) || g.a_bf16 != gs[first].a_bf16 || g.c_bf16 != gs[first].c_bf16) {
                set_error("gemm_bf16_batched: unsupported shape M=%lld N=%d K=%d (or mixed operand types)",
                          (long long)g.M, g.N, g.K);
                return false;
            }
            b.d[i] = to_desc_bf16(g);
            max_tiles = std::max(max_tiles, tiles_bf16(g));
            dma = dma && dma_ok(g);
        }
        if (!launch_bf16(s, epilogue, gs[first].a_bf16, gs[first].c_bf16, nullptr, &b, (unsigned)max_tiles,
                         (unsigned)count, dma))
            return false;
    }
    return true;
}

// ------------------------------------------------------------ split GEMM
static_assert(GS_BK == SPLIT_K_MULTIPLE, "split GEMM K chunk");

static bool gemm_split_ok(const GemmArgsSplit &g, int epilogue) {
    if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.M > INT32_MAX / 2) return false;
    if (g.K % GS_BK || g.lda % 4 || g.lda < g.K || g.lda > (1 << 21)) return false;  // lane load offsets are 32-bit
    // the epilogue's row offsets within a wave's rows are 32-bit
    if (g.ldc < out_cols(g.N, epilogue) || g.ldc > (1 << 21) || (epilogue == EPI_GEGLU && g.N % 64)) return false;
    if (((uintptr_t)g.A | (uintptr_t)g.W) & 15) return false;
    return true;
}

static GemmDescSplit to_desc_split(const GemmArgsSplit &g) {
    GemmDescSplit d;
    d.A = g.A; d.W = static_cast<const bf16 *>(g.W); d.bias = g.bias; d.C = g.C;
    d.M = (int)g.M; d.N = g.N; d.K = g.K;
    d.lda = g.lda; d.ldc = g.ldc;
    return d;
}

template <int EPI>
static void launch_split(hipStream_t s, const GemmDescSplit &d, unsigned tiles) {
    hipLaunchKernelGGL(gemm_split_kernel<EPI>, dim3(tiles), dim3(GS_THREADS), 0, s, d);
}

bool gemm_split(hipStream_t s, const GemmArgsSplit &g, int epilogue, KernelTimer *t, const char *name) {
    if (!gemm_split_ok(g, epilogue)) {
        set_error("gemm_split: unsupported shape M=%lld N=%d K=%d lda=%d", (long long)g.M, g.N, g.K, g.lda);
        return false;
    }
    const GemmDescSplit d = to_desc_split(g);
    const unsigned tiles = (unsigned)(((g.M + GS_BM - 1) / GS_BM) * ((g.N + GS_BN - 1) / GS_BN));
    Scope sc(t, s, name);
    switch (epilogue) {
        case EPI_STORE: launch_split<EPI_STORE>(s, d, tiles); break;
        case EPI_GELU: launch_split<EPI_GELU>(s, d, tiles); break;
        case EPI_TANH: launch_split<EPI_TANH>(s, d, tiles); break;
        case EPI_RESIDUAL: launch_split<EPI_RESIDUAL>(s, d, tiles); break;
        case EPI_GEGLU: launch_split<EPI_GEGLU>(s, d, tiles); break;
        default: set_error("unknown GEMM epilogue %d", epilogue); return false;
    }
    return sync_debug(s, "gemm_split_kernel");
}

bool split_weights(hipStream_t s, const float *W, int N, int K, int ldw, void *pieces) {
    if (N <= 0 || K <= 0 || K % GS_BK || ldw < K || split_bytes(N, K) / 6 > (size_t)INT32_MAX) {
        set_error("split_weights: bad shape N=%d K=%d ldw=%d (K a multiple of 16)", N, K, ldw);
        return false;
    }
    const int64_t n = (int64_t)(N + GS_BN - 1) / GS_BN * GS_BN * K;
    hipLaunchKernelGGL(split_weight_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, W, N, K, ldw,
                       static_cast<bf16 *>(pieces));
    return sync_debug(s, "split_weight_kernel");
}

// ------------------------------------------------------- fp16 two-piece GEMM
static bool gemm_h2_ok(const GemmArgsH2 &g, int epilogue) {
    if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.M > INT32_MAX / 2 || !g.W) return false;
    if (g.K % GS_BK || g.lda % 4 || g.lda < g.K || g.lda > (1 << 21)) return false;  // lane load offsets are 32-bit
    // the epilogue's row offsets within a wave's rows are 32-bit
    if (g.ldc < out_cols(g.N, epilogue) || g.ldc > (1 << 21) || (epilogue == EPI_GEGLU && g.N % 64)) return false;
    if (((uintptr_t)g.A | (uintptr_t)g.W) & 15) return false;
    if (g.row_norm && (g.a_h2 || !(epilogue == EPI_STORE || epilogue == EPI_GELU || epilogue == EPI_GEGLU)))
        return false;
    if (g.amax && epilogue != EPI_RESIDUAL) return false;
    if (g.kv_inner && (g.kv_inner < 0 || g.kv_inner % 32 || !g.kv_bound || epilogue != EPI_STORE || !g.row_norm))
        return false;
    if (g.kv_pieces && (!g.kv_inner || g.kv_inner % 128 || !g.rope || g.rope_period <= 0 || g.rope_len <= 0 ||
                        3 * g.kv_inner > g.N))
        return false;
    return true;
}

static GemmDescH2 to_desc_h2(const GemmArgsH2 &g) {
    GemmDescH2 d;
    d.A = g.A; d.W = g.W; d.bias = g.bias; d.C = g.C;
    d.M = (int)g.M; d.N = g.N; d.K = g.K;
    d.lda = g.lda; d.ldc = g.ldc;
    d.zero_slot = g.zero_slot; d.amax = g.amax;
    d.kv_bound = g.kv_bound; d.kv_inner = g.kv_inner;
    d.kv_pieces = g.kv_pieces ? 1 : 0;
    d.rope = g.rope; d.rope_period = g.rope_period; d.rope_len = g.rope_len;
    return d;
}

template <int EPI>
static void launch_h2(hipStream_t s, const GemmDescH2 &d, const H2Bound &b, unsigned tiles, const GemmArgsH2 &g) {
    if constexpr (EPI == EPI_STORE || EPI == EPI_GELU || EPI == EPI_GEGLU) {
        if (g.row_norm) {  // gemm_h2_ok: fp32 A
            if constexpr (EPI == EPI_STORE) {
                if (g.kv_inner) {  // the fused projection with k and v scaled
                    hipLaunchKernelGGL((gemm_h2_kernel<EPI, false, true, true>), dim3(tiles), dim3(GS_THREADS), 0, s,
                                       d, b);
                    return;
                }
            }
            hipLaunchKernelGGL((gemm_h2_kernel<EPI, false, true>), dim3(tiles), dim3(GS_THREADS), 0, s, d, b);
            return;
        }
    }
    if (g.a_h2) hipLaunchKernelGGL((gemm_h2_kernel<EPI, true>), dim3(tiles), dim3(GS_THREADS), 0, s, d, b);
    else hipLaunchKernelGGL((gemm_h2_kernel<EPI, false>), dim3(tiles), dim3(GS_THREADS), 0, s, d, b);
}

bool gemm_h2(hipStream_t s, const GemmArgsH2 &g, const OperandBound &bound, int epilogue, KernelTimer *t,
             const char *name) {
    if (!gemm_h2_ok(g, epilogue)) {
        set_error("gemm_h2: unsupported shape or mode M=%lld N=%d K=%d lda=%d epilogue %d%s%s", (long long)g.M, g.N,
                  g.K, g.lda, epilogue, g.row_norm ? " row norm" : "", g.amax ? " amax" : "");
        return false;
    }
    // every workgroup reads the bound as it starts, while tile 0 zeroes
    // zero_slot and the epilogues raise amax: neither may be the bound
    if (bound.dev && (g.zero_slot == bound.dev || g.amax == bound.dev)) {
        set_error("gemm_h2: zero_slot and amax must not alias the A bound");
        return false;
    }
    const GemmDescH2 d = to_desc_h2(g);
    const H2Bound b{bound.dev, bound.value};
    const unsigned tiles = (unsigned)(((g.M + GS_BM - 1) / GS_BM) * ((g.N + GS_BN - 1) / GS_BN));
    Scope sc(t, s, name);
    switch (epilogue) {
        case EPI_STORE: launch_h2<EPI_STORE>(s, d, b, tiles, g); break;
        case EPI_GELU: launch_h2<EPI_GELU>(s, d, b, tiles, g); break;
        case EPI_TANH: launch_h2<EPI_TANH>(s, d, b, tiles, g); break;
        case EPI_RESIDUAL: launch_h2<EPI_RESIDUAL>(s, d, b, tiles, g); break;
        case EPI_GEGLU: launch_h2<EPI_GEGLU>(s, d, b, tiles, g); break;
        default: set_error("unknown GEMM epilogue %d", epilogue); return false;
    }
    return sync_debug(s, "gemm_h2_kernel");
}

bool band_attention(hipStream_t s, const BandAttention &b, KernelTimer *t) {
    const int inner = b.heads * ATT_DH;
    // a tile's rows (two sequences) lie within 2^32 bytes of its first row
    const bool ok = b.x && b.W && b.out && b.x_bound && b.bound && b.rope && b.S > 0 && b.L > 0 && b.L <= 64 && b.heads > 0 &&
                    b.K >= GS_BK && b.K % GS_BK == 0 && b.K <= BA_MAX_K && b.lda >= b.K && b.lda % 4 == 0 &&
                    b.lda <= (1 << 21) && inner % GS_BN == 0 && b.ld_out >= inner && b.ld_out % 4 == 0 &&
                    (int64_t)b.S * b.L <= INT32_MAX / 2 && !(((uintptr_t)b.x | (uintptr_t)b.W | (uintptr_t)b.out) & 15) &&
                    !((uintptr_t)b.gate_w & 15);
    if (!ok) {
        set_error("band_attention: unsupported shape S=%d L=%d heads=%d K=%d lda=%d ld_out=%d", b.S, b.L, b.heads, b.K,
                  b.lda, b.ld_out);
        return false;
    }
    // every workgroup reads x while others write out: the two must not overlap
    const uintptr_t x0 = (uintptr_t)b.x, x1 = x0 + (uintptr_t)((int64_t)b.S * b.L * b.lda * sizeof(float));
    const uintptr_t o0 = (uintptr_t)b.out, o1 = o0 + (uintptr_t)((int64_t)b.S * b.L * b.ld_out * sizeof(float));
    if (o0 < x1 && x0 < o1) {
        set_error("band_attention: out overlaps x");
        return false;
    }
    BandAttnArgs a;
    a.x = b.x; a.lda = b.lda; a.K = b.K;
    a.W = b.W; a.bias = b.bias; a.gate_w = b.gate_w; a.gate_b = b.gate_b;
    a.x_bound = b.x_bound; a.bound = b.bound; a.rope = b.rope;
    a.out = b.out; a.ld_out = b.ld_out;
    a.S = b.S; a.L = b.L; a.H = b.heads;
    a.scale = 0.125f;
    const unsigned grid = (unsigned)(((int64_t)b.S + 1) / 2 * b.heads);
    Scope sc(t, s, "band_attention");
    hipLaunchKernelGGL(band_attention_fused_kernel, dim3(grid), dim3(BA_THREADS), 0, s, a);
    return sync_debug(s, "band_attention_fused_kernel");
}

template <int EPI>
static void launch_h2_batched(hipStream_t s, const GemmBatchH2 &b, unsigned tiles, unsigned n) {
    hipLaunchKernelGGL(gemm_h2_batched_kernel<EPI>, dim3(tiles, 1, n), dim3(GS_THREADS), 0, s, b);
}

bool gemm_h2_batched(hipStream_t s, const std::vector<GemmArgsH2> &gs, const OperandBound &bound, int epilogue,
                     KernelTimer *t, const char *name) {
    Scope sc(t, s, name);
    for (size_t first = 0; first < gs.size(); first += GS_MAX_BATCH) {
        const size_t count = std::min(gs.size() - first, (size_t)GS_MAX_BATCH);
        GemmBatchH2 b;
        memset(&b, 0, sizeof(b));
        b.b = H2Bound{bound.dev, bound.value};
        int64_t max_tiles = 0;
        for (size_t i = 0; i < count; i++) {
            const GemmArgsH2 &g = gs[first + i];
            if (!gemm_h2_ok(g, epilogue)) {
                set_error("gemm_h2_batched: unsupported shape M=%lld N=%d K=%d lda=%d", (long long)g.M, g.N, g.K,
                          g.lda);
                return false;
            }
            // the batched kernel splits fp32 A and has none of the single
            // GEMM's modes
            if (g.row_norm || g.a_h2 || g.kv_inner || g.zero_slot || g.amax) {
                set_error("gemm_h2_batched: row_norm, a_h2, kv_inner, zero_slot and amax are not supported");
                return false;
            }
            b.d[i] = to_desc_h2(g);
            max_tiles = std::max(max_tiles, ((g.M + GS_BM - 1) / GS_BM) * ((g.N + GS_BN - 1) / GS_BN));
        }
        const unsigned tiles = (unsigned)max_tiles, n = (unsigned)count;
        switch (epilogue) {
            case EPI_STORE: launch_h2_batched<EPI_STORE>(s, b, tiles, n); break;
            case EPI_GELU: launch_h2_batched<EPI_GELU>(s, b, tiles, n); break;
            case EPI_TANH: launch_h2_batched<EPI_TANH>(s, b, tiles, n); break;
            case EPI_RESIDUAL: launch_h2_batched<EPI_RESIDUAL>(s, b, tiles, n); break;
            case EPI_GEGLU: launch_h2_batched<EPI_GEGLU>(s, b, tiles, n); break;
            default: set_error("unknown GEMM epilogue %d", epilogue); return false;
        }
        if (!sync_debug(s, "gemm_h2_batched_kernel")) return false;
    }
    return true;
}

bool split_weights_h2(hipStream_t s, const float *W, int N, int K, int ldw, void *pieces) {
    if (N <= 0 || K <= 0 || K % GS_BK || ldw < K || (h2_bytes(N, K) - H2_HEADER) / 4 > (size_t)INT32_MAX ||
        ((uintptr_t)pieces & 255)) {
        set_error("split_weights_h2: bad shape N=%d K=%d ldw=%d (K a multiple of 16, pieces 256-byte aligned)", N, K,
                  ldw);
        return false;
    }
    hipLaunchKernelGGL(zero_float_kernel, dim3(1), dim3(1), 0, s, static_cast<float *>(pieces));
    const int64_t nw = (int64_t)N * K;
    hipLaunchKernelGGL(absmax_rows_kernel, dim3((unsigned)std::min<int64_t>(512, (nw + 4095) / 4096)), dim3(256), 0, s,
                       W, N, K, ldw, static_cast<float *>(pieces));
    if (!sync_debug(s, "absmax_rows_kernel")) return false;
    const int64_t n = (int64_t)(N + GS_BN - 1) / GS_BN * GS_BN * K;
    hipLaunchKernelGGL(split_weight_h2_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, W, N, K, ldw, pieces);
    return sync_debug(s, "split_weight_h2_kernel");
}

bool absmax(hipStream_t s, const float *x, int64_t n, float *scratch, float *out) {
    if (!x || n <= 0 || !scratch || !out) {
        set_error("absmax: bad arguments");
        return false;
    }
    const unsigned blocks = (unsigned)std::min<int64_t>(ABSMAX_PARTIALS, (n + 1023) / 1024);
    hipLaunchKernelGGL(absmax_partial_kernel, dim3(blocks), dim3(256), 0, s, x, n, scratch);
    if (!sync_debug(s, "absmax_partial_kernel")) return false;
    hipLaunchKernelGGL(absmax_kernel, dim3(1), dim3(1024), 0, s, scratch, 1, (int)blocks, (int)blocks, out);
    return sync_debug(s, "absmax_kernel");
}

bool layer_bounds(hipStream_t s, const Dims &d, const LayerWeights &w, float *bounds) {
    // bounds[1] covers the q, k, v rows of the fused projection only (their
    // bias is zero): it scales q, k, v in the attention and bounds the
    // attention output; the gate logits pass through a sigmoid
    return operand_bounds(s, w.gamma, d.dim, w.wqkvg, d.qkv_dim(), w.bqkvg, false, bounds) &&
           operand_bounds(s, w.ff_gamma, d.dim, w.w1, d.ff1_out(), w.b1, d.ffn_glu != 0, bounds + 2);
}

int bounds_usable(hipStream_t s, const float *dev, int n, float *host) {
    float h[8];
    if (n > 8 || !check(hipMemcpyAsync(h, dev, n * sizeof(float), hipMemcpyDeviceToHost, s), "hipMemcpy(bounds)") ||
        !check(hipStreamSynchronize(s), "hipStreamSynchronize(bounds)"))
        return -1;
    if (host) memcpy(host, h, n * sizeof(float));
    for (int i = 0; i < n; i++)
        if (!(h[i] >= 0.0f && h[i] <= 1.0e30f)) return 0;  // NaN, infinite or beyond the scale range
    return 1;
}

bool operand_bounds(hipStream_t s, const float *gamma, int D, const float *W, int N, const float *b, bool square,
                    float *out) {
    if (!gamma || D <= 0 || (W && N <= 0) || !out) {
        set_error("operand_bounds: bad arguments D=%d N=%d", D, N);
        return false;
    }
    hipLaunchKernelGGL(operand_bounds_kernel, dim3(1), dim3(1024), 0, s, gamma, D, W, N, b, square ? 1 : 0, out);
    return sync_debug(s, "operand_bounds_kernel");
}

bool to_bf16_rows(hipStream_t s, const float *src, int rows, int cols, void *dst, int ld) {
    const int64_t n = (int64_t)rows * cols;
    hipLaunchKernelGGL(to_bf16_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, src, static_cast<bf16 *>(dst),
                       (int64_t)rows, cols, ld);
    return sync_debug(s, "to_bf16_kernel");
}

// Rows of x and y are contiguous (pitch dim): the kernels take rows in pairs
// as one span.
template <typename TY>
static bool rmsnorm_any(hipStream_t s, const float *x, int ldx, const float *gamma, TY *y, int ldy, int64_t rows,
                        int dim, KernelTimer *t) {
    if (dim % 4 || dim > 2048 || rows <= 0 || rows > INT32_MAX / 2 || ldx != dim || ldy != dim) {
        set_error("rmsnorm: unsupported dim %d or row pitches %d/%d", dim, ldx, ldy);
        return false;
    }
    Scope sc(t, s, "rmsnorm");
    const unsigned grid = blocks_for((rows + 1) / 2, 4);
    const int nv2 = dim / 2;  // float4s of a pair
    if (nv2 <= 64) hipLaunchKernelGGL((rmsnorm_kernel<1, TY>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim);
    else if (nv2 <= 128) hipLaunchKernelGGL((rmsnorm_kernel<2, TY>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim);
    else if (nv2 <= 192) hipLaunchKernelGGL((rmsnorm_kernel<3, TY>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim);
    else if (nv2 <= 256) hipLaunchKernelGGL((rmsnorm_kernel<4, TY>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim);
    else if (nv2 <= 512) hipLaunchKernelGGL((rmsnorm_kernel<8, TY>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim);
    else hipLaunchKernelGGL((rmsnorm_kernel<16, TY>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim);
    return sync_debug(s, "rmsnorm_kernel");
}

bool rmsnorm_h2(hipStream_t s, const float *x, int ldx, const float *gamma, float *y, int ldy, int64_t rows, int dim,
                const float *bound, KernelTimer *t) {
    if (dim % 16 || dim > 2048 || rows <= 0 || rows > INT32_MAX / 2 || !bound || ldx != dim || ldy != dim) {
        set_error("rmsnorm_h2: unsupported dim %d or row pitches %d/%d", dim, ldx, ldy);
        return false;
    }
    Scope sc(t, s, "rmsnorm");
    const unsigned grid = blocks_for((rows + 1) / 2, 4);
    const int nv2 = dim / 2;
    if (nv2 <= 64) hipLaunchKernelGGL((rmsnorm_h2_kernel<1>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim, bound);
    else if (nv2 <= 128) hipLaunchKernelGGL((rmsnorm_h2_kernel<2>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim, bound);
    else if (nv2 <= 192) hipLaunchKernelGGL((rmsnorm_h2_kernel<3>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim, bound);
    else if (nv2 <= 256) hipLaunchKernelGGL((rmsnorm_h2_kernel<4>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim, bound);
    else if (nv2 <= 512) hipLaunchKernelGGL((rmsnorm_h2_kernel<8>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim, bound);
    else hipLaunchKernelGGL((rmsnorm_h2_kernel<16>), dim3(grid), dim3(256), 0, s, x, gamma, y, (int)rows, dim, bound);
    return sync_debug(s, "rmsnorm_h2_kernel");
}

bool rmsnorm(hipStream_t s, const float *x, int ldx, const float *gamma, float *y, int ldy, int64_t rows, int dim,
             KernelTimer *t) {
    return rmsnorm_any<float>(s, x, ldx, gamma, y, ldy, rows, dim, t);
}

bool rmsnorm_bf16(hipStream_t s, const float *x, int ldx, const float *gamma, void *y, int ldy, int64_t rows, int dim,
                  KernelTimer *t) {
    return rmsnorm_any<bf16>(s, x, ldx, gamma, static_cast<bf16 *>(y), ldy, rows, dim, t);
}

bool softmax_rows(hipStream_t s, const float *in, float *out, int64_t rows, int len, KernelTimer *t) {
    if (len <= 0 || len > 4 * 64 * 16 - 4 || (((uintptr_t)in | (uintptr_t)out) & 15)) {
        set_error("softmax_rows: unsupported length %d or unaligned buffers", len);
        return false;
    }
    Scope sc(t, s, "softmax");
    const unsigned grid = blocks_for(rows, 4);
    const size_t lds = 4 * (size_t)len * sizeof(float);
    if (len <= 256) hipLaunchKernelGGL(softmax_rows_kernel<4>, dim3(grid), dim3(256), lds, s, in, out, rows, len);
    else if (len <= 512) hipLaunchKernelGGL(softmax_rows_kernel<8>, dim3(grid), dim3(256), lds, s, in, out, rows, len);
    else if (len <= 832) hipLaunchKernelGGL(softmax_rows_kernel<13>, dim3(grid), dim3(256), lds, s, in, out, rows, len);
    else if (len <= 1024) hipLaunchKernelGGL(softmax_rows_kernel<16>, dim3(grid), dim3(256), lds, s, in, out, rows, len);
    else if (len <= 2048) hipLaunchKernelGGL(softmax_rows_kernel<32>, dim3(grid), dim3(256), lds, s, in, out, rows, len);
    else hipLaunchKernelGGL(softmax_rows_kernel<64>, dim3(grid), dim3(256), lds, s, in, out, rows, len);
    return sync_debug(s, "softmax_rows_kernel");
}

bool rope_bhld(hipStream_t s, float *x, const float *cs, const float *sn, int64_t bh, int len, KernelTimer *t) {
    const int64_t n4 = bh * len * 16;
    Scope sc(t, s, "rope");
    hipLaunchKernelGGL(rope_bhld_kernel, dim3(blocks_for(n4, 256)), dim3(256), 0, s, x, cs, sn, n4, len);
    return sync_debug(s, "rope_bhld_kernel");
}

bool geglu(hipStream_t s, const float *in, float *out, int64_t rows, int width, KernelTimer *t) {
    if (width % 4) {
        set_error("geglu: width %% 4 != 0");
        return false;
    }
    Scope sc(t, s, "geglu");
    hipLaunchKernelGGL(geglu_kernel, dim3(blocks_for(rows * (width / 4), 256)), dim3(256), 0, s, in, out, rows, width);
    return sync_debug(s, "geglu_kernel");
}

bool residual_add(hipStream_t s, float *x, const float *r, int64_t n, KernelTimer *t) {
    if (n % 4) {
        set_error("residual_add: n %% 4 != 0");
        return false;
    }
    Scope sc(t, s, "residual");
    hipLaunchKernelGGL(residual_add_kernel, dim3(blocks_for(n / 4, 256)), dim3(256), 0, s, x, r, n / 4);
    return sync_debug(s, "residual_add_kernel");
}

bool unpack_weight(hipStream_t s, const float *packed_dev, int in, int out, float *dst, int ldd, int row0, int mode) {
    hipLaunchKernelGGL(unpack_weight_kernel, dim3(blocks_for((int64_t)in * out, 256)), dim3(256), 0, s, packed_dev, in,
                       out, dst, ldd, row0, mode);
    return sync_debug(s, "unpack_weight_kernel");
}

bool fold_gain_split_h2(hipStream_t s, const float *W, int N, int K, int ldw, const float *gamma, float *tmp,
                        void *pieces) {
    if (!W || !gamma || !tmp || N <= 0 || K <= 0 || ldw < K) {
        set_error("fold_gain_split_h2: bad arguments N=%d K=%d ldw=%d", N, K, ldw);
        return false;
    }
    const int64_t n = (int64_t)N * K;
    hipLaunchKernelGGL(scale_columns_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, W, N, K, ldw, gamma, tmp);
    if (!sync_debug(s, "scale_columns_kernel")) return false;
    return split_weights_h2(s, tmp, N, K, K, pieces);
}

bool interleave_glu_bias(hipStream_t s, const float *src, float *dst, int out) {
    hipLaunchKernelGGL(interleave_glu_bias_kernel, dim3(blocks_for(out, 256)), dim3(256), 0, s, src, dst, out);
    return sync_debug(s, "interleave_glu_bias_kernel");
}

bool transpose_rows(hipStream_t s, const float *src, float *dst, int outer, int a, int b, int dim) {
    if (dim % 4) {
        set_error("transpose_rows: dim %% 4 != 0");
        return false;
    }
    const int64_t n = (int64_t)outer * a * b * (dim / 4);
    hipLaunchKernelGGL(transpose_rows_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, src, dst, outer, a, b, dim / 4);
    return sync_debug(s, "transpose_rows_kernel");
}

template <int WAVES>
static void launch_attention(hipStream_t s, const AttnArgs &a, unsigned grid, bool out_bf16, bool qkv_bf16,
                             bool split) {
    const dim3 block(64 * WAVES);
    if constexpr (WAVES == 4) {
        if (split) {
            // 32-bit staging offsets when the last row's end lies below 4 GB
            // and one position step below 16 MB (positive strides)
            const int64_t last_row = (int64_t)((a.S - 1) / a.group) * a.group_stride +
                                     (int64_t)(std::min(a.S, a.group) - 1) * a.seq_stride +
                                     (int64_t)(a.L - 1) * a.pos_stride;
            const bool off32 = a.group_stride >= 0 && a.seq_stride >= 0 && a.pos_stride >= 0 &&
                               (last_row + 1) * a.ld * 4 <= (int64_t)UINT32_MAX &&
                               (int64_t)a.pos_stride * a.ld * 4 < (1 << 24);
            auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, dim3(grid), block, 0, s, a); };
            if (a.kv_pieces) {  // attention() checked off32
                go(attention_h2_kvp_kernel<WAVES>);
                return;
            }
            if (a.bound && a.kv_scaled) {  // fp16 two-piece products, k and v prescaled (fp32 out)
                if (a.rope) off32 ? go(attention_h2_kernel<WAVES, float, true, true, true>)
                                  : go(attention_h2_kernel<WAVES, float, true, false, true>);
                else off32 ? go(attention_h2_kernel<WAVES, float, false, true, true>)
                           : go(attention_h2_kernel<WAVES, float, false, false, true>);
                return;
            }
            if (a.bound) {  // fp16 two-piece products
                if (a.rope) {
                    if (out_bf16) off32 ? go(attention_h2_kernel<WAVES, bf16, true, true>)
                                        : go(attention_h2_kernel<WAVES, bf16, true, false>);
                    else off32 ? go(attention_h2_kernel<WAVES, float, true, true>)
                               : go(attention_h2_kernel<WAVES, float, true, false>);
                } else {
                    if (out_bf16) off32 ? go(attention_h2_kernel<WAVES, bf16, false, true>)
                                        : go(attention_h2_kernel<WAVES, bf16, false, false>);
                    else off32 ? go(attention_h2_kernel<WAVES, float, false, true>)
                               : go(attention_h2_kernel<WAVES, float, false, false>);
                }
                return;
            }
            if (a.rope) {
                if (out_bf16) off32 ? go(attention_split_kernel<WAVES, bf16, true, true>)
                                    : go(attention_split_kernel<WAVES, bf16, true, false>);
                else off32 ? go(attention_split_kernel<WAVES, float, true, true>)
                           : go(attention_split_kernel<WAVES, float, true, false>);
            } else {
                if (out_bf16) off32 ? go(attention_split_kernel<WAVES, bf16, false, true>)
                                    : go(attention_split_kernel<WAVES, bf16, false, false>);
                else off32 ? go(attention_split_kernel<WAVES, float, false, true>)
                           : go(attention_split_kernel<WAVES, float, false, false>);
            }
            return;
        }
    }
    if (qkv_bf16) {
        if (out_bf16) hipLaunchKernelGGL((attention_bf16_kernel<WAVES, bf16>), dim3(grid), block, 0, s, a);
        else hipLaunchKernelGGL((attention_bf16_kernel<WAVES, float>), dim3(grid), block, 0, s, a);
    } else {
        if (out_bf16) hipLaunchKernelGGL((attention_kernel<WAVES, bf16>), dim3(grid), block, 0, s, a);
        else hipLaunchKernelGGL((attention_kernel<WAVES, float>), dim3(grid), block, 0, s, a);
    }
}

bool attention(hipStream_t s, const void *qkv, int ld, void *out, int ld_out, const float *rope, const AttnLayout &lay,
               int heads, int gate_col, KernelTimer *t, bool out_bf16, bool qkv_bf16, bool split, const float *bound,
               bool out_h2, bool kv_scaled, bool device_choice, bool kv_pieces) {
    if (lay.S <= 0 || lay.L <= 0 || ld % (qkv_bf16 ? 8 : 4) || ld_out % 4 || ((uintptr_t)qkv & 15)) {
        set_error("attention: bad shape S=%d L=%d ld=%d", lay.S, lay.L, ld);
        return false;
    }
    if (out_h2 && (out_bf16 || qkv_bf16 || !split || !bound || ((uintptr_t)out & 15))) {
        set_error("attention: h2 rows out need the fp16 two-piece kernels (fp32 qkv, a bound) and a 16-byte aligned out");
        return false;
    }
    if (kv_scaled && (out_bf16 || qkv_bf16 || !split || !bound)) {
        set_error("attention: prescaled k and v need the fp16 two-piece kernels (fp32 qkv and out, a bound)");
        return false;
    }
    if (kv_pieces) {
        // the DMA staging's 32-bit offsets from a sequence's first row
        const int64_t last_row = (int64_t)((lay.S - 1) / lay.group) * lay.group_stride +
                                 (int64_t)(std::min(lay.S, lay.group) - 1) * lay.seq_stride +
                                 (int64_t)(lay.L - 1) * lay.pos_stride;
        const bool off32 = lay.group_stride >= 0 && lay.seq_stride >= 0 && lay.pos_stride >= 0 &&
                           (last_row + 1) * ld * 4 <= (int64_t)UINT32_MAX;
        if (!kv_scaled || lay.L <= 64 || !rope || heads * ATT_DH % 128 || device_choice || out_bf16 || !off32) {
            set_error("attention: k/v pieces need the prescaled two-piece kernel, L > 64, fp32 out, the rotary "
                      "table and 32-bit staging offsets");
            return false;
        }
    }
    if (device_choice && (qkv_bf16 || !split || !bound || out_h2 || kv_scaled)) {
        set_error("attention: the device-side range choice needs fp32 qkv, split and a bound, without h2 or "
                  "prescaled operands");
        return false;
    }
    AttnArgs a;
    a.qkv = qkv; a.ld = ld; a.out = out; a.ld_out = ld_out;
    a.rope = rope;
    a.S = lay.S; a.L = lay.L; a.H = heads;
    a.group = lay.group; a.group_stride = lay.group_stride; a.seq_stride = lay.seq_stride; a.pos_stride = lay.pos_stride;
    a.inner = heads * ATT_DH; a.gate_col = gate_col; a.scale = 0.125f;
    a.bound = split && !qkv_bf16 ? bound : nullptr;
    a.out_h2 = out_h2 ? 1 : 0;
    a.kv_scaled = kv_scaled ? 1 : 0;
    a.guard = nullptr;
    a.guard_h2 = 0;
    a.kv_pieces = kv_pieces ? 1 : 0;
    Scope sc(t, s, lay.L > 64 ? "attention_long" : "attention_short");
    auto launch = [&](const AttnArgs &a) {
        if (lay.L <= 64 && !qkv_bf16) {
            // persistent: four workgroups per CU loop over the (sequence, head) tasks
            static int cus = 0;
            if (cus == 0 && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess)
                cus = 256;
            const unsigned grid = (unsigned)std::min<int64_t>((int64_t)lay.S * heads, 4 * (int64_t)cus);
            if (a.bound) {  // fp16 two-piece products
                if (out_bf16) hipLaunchKernelGGL((attention_short_h2_kernel<bf16>), dim3(grid), dim3(256), 0, s, a);
                else if (kv_scaled)
                    hipLaunchKernelGGL((attention_short_h2_kernel<float, true>), dim3(grid), dim3(256), 0, s, a);
                else hipLaunchKernelGGL((attention_short_h2_kernel<float>), dim3(grid), dim3(256), 0, s, a);
            } else if (out_bf16) hipLaunchKernelGGL((attention_short_kernel<bf16>), dim3(grid), dim3(256), 0, s, a);
            else hipLaunchKernelGGL((attention_short_kernel<float>), dim3(grid), dim3(256), 0, s, a);
        } else if (lay.L <= 64)
            launch_attention<2>(s, a, (unsigned)((int64_t)lay.S * heads * ((lay.L + 63) / 64)), out_bf16, qkv_bf16,
                                split && !qkv_bf16);
        else launch_attention<4>(s, a, (unsigned)((int64_t)lay.S * heads * ((lay.L + 127) / 128)), out_bf16, qkv_bf16,
                                 split && !qkv_bf16);
    };
    if (device_choice) {
        // the two-piece kernel when the bound is in range, else the kernel
        // without piece scales (three-piece bf16 for L > 64, fp32 MFMA below)
        AttnArgs in = a, out_of = a;
        in.guard = bound;
        in.guard_h2 = 1;
        out_of.bound = nullptr;
        out_of.guard = bound;
        out_of.guard_h2 = 0;
        launch(in);
        if (!sync_debug(s, "attention_kernel (bound in range)")) return false;
        launch(out_of);
    } else {
        launch(a);
    }
    return sync_debug(s, "attention_kernel");
}

// ------------------------------------------------------------------- dims
Dims dims_from(const vh_dims &d) {
    Dims o;
    o.dim = d.dim; o.depth = d.depth; o.bands = d.bands; o.heads = d.heads; o.dim_head = d.dim_head;
    o.ff_dim = d.ff_dim; o.ffn_glu = d.ffn_glu; o.gated = d.gated; o.mask_hidden = d.mask_hidden;
    o.n_fft = d.n_fft; o.hop = d.hop; o.channels = d.channels;
    for (int i = 0; i < VH_MAX_BANDS; i++) o.band_widths[i] = i < d.bands ? d.band_widths[i] : 0;
    return o;
}

bool Dims::valid(char *why, size_t n) const {
    if (dim_head != 64) { snprintf(why, n, "dim_head must be 64 (got %d)", dim_head); return false; }
    if (dim <= 0 || dim % 4 || dim > 2048) { snprintf(why, n, "dim must be a multiple of 4 up to 2048"); return false; }
    if (heads <= 0 || bands <= 0 || bands > VH_MAX_BANDS || depth < 0) { snprintf(why, n, "bad heads/bands/depth"); return false; }
    if (ffn_glu && (ff_dim % 32)) { snprintf(why, n, "GELU-GLU needs ff_dim %% 32 == 0"); return false; }
    if (ff_dim % 4 || mask_hidden % 4 || mask_hidden <= 0) { snprintf(why, n, "ff_dim/mask_hidden must be multiples of 4"); return false; }
    if (n_fft <= 0 || (n_fft & (n_fft - 1)) || n_fft > 4096 || hop <= 0) { snprintf(why, n, "n_fft must be a power of two <= 4096"); return false; }
    if (channels <= 0 || channels > 8) { snprintf(why, n, "bad channel count"); return false; }
    int sum = 0;
    for (int b = 0; b < bands; b++) {
        if (band_widths[b] <= 0 || band_widths[b] * channels > 320) { snprintf(why, n, "band %d too wide", b); return false; }
        sum += band_widths[b];
    }
    if (sum != freq_bins()) { snprintf(why, n, "band widths sum to %d, expected %d", sum, freq_bins()); return false; }
    return true;
}

// ------------------------------------------------------------------ rotary
void rope_table_host(int length, int dim_head, float *cos_t, float *sin_t, float *interleaved) {
    const int pairs = dim_head / 2;
    std::vector<float> freq(pairs > 0 ? pairs : 0);
    for (int i = 0; i < pairs; i++) freq[i] = 1.0f / powf(10000.0f, (float)(2 * i) / (float)dim_head);
    for (int p = 0; p < length; p++)
        for (int k = 0; k < pairs; k++) {
            const float angle = (float)p * freq[k];
            const size_t e = (size_t)p * pairs + k;
            const float c = cosf(angle), sn = sinf(angle);
            if (cos_t) cos_t[e] = c;
            if (sin_t) sin_t[e] = sn;
            if (interleaved) {
                interleaved[2 * e] = c;
                interleaved[2 * e + 1] = sn;
            }
        }
}

bool RopeCache::get(int length, int dim_head, hipStream_t s, const float **cs, const float **sn) {
    auto it = tables.find(length);
    if (it == tables.end()) {
        const int pairs = dim_head / 2;
        const size_t n = (size_t)length * pairs;
        std::vector<float> h(4 * n);
        float *hc = h.data(), *hs = hc + n, *hi = hs + n;
        rope_table_host(length, dim_head, hc, hs, hi);
        float *d = nullptr;
        const size_t bytes = h.size() * sizeof(float);
        if (!check(hipMalloc((void **)&d, bytes), "hipMalloc(rope tables)")) return false;
        if (!check(hipMemcpyAsync(d, h.data(), bytes, hipMemcpyHostToDevice, s), "hipMemcpy(rope tables)") ||
            !check(hipStreamSynchronize(s), "hipStreamSynchronize(rope)")) {
            (void)hipFree(d);
            return false;
        }
        it = tables.emplace(length, Tables{d, d + n, d + 2 * n}).first;
    }
    *cs = it->second.cos;
    *sn = it->second.sin;
    return true;
}

bool RopeCache::get_interleaved(int length, int dim_head, hipStream_t s, const float **cssn) {
    const float *cs, *sn;
    if (!get(length, dim_head, s, &cs, &sn)) return false;
    *cssn = tables[length].interleaved;
    return true;
}

void RopeCache::release() {
    for (auto &kv : tables) (void)hipFree(kv.second.cos);  // one allocation per length
    tables.clear();
}

// --------------------------------------------------------------- block
bool BlockScratch::ensure(const Dims &d, int64_t tokens) {
    const size_t t = (size_t)tokens;
    return normed.ensure(t * d.dim * sizeof(float), "hipMalloc(normed)") &&
           qkvg.ensure(t * d.qkvg_dim() * sizeof(float), "hipMalloc(qkv)") &&
           attn.ensure(t * d.inner() * sizeof(float), "hipMalloc(attention)") &&
           hidden.ensure(t * d.ff_dim * sizeof(float), "hipMalloc(ffn hidden)");
}

bool transformer_block(hipStream_t s, const Dims &d, const LayerWeights &w, float *x, int64_t tokens,
                       const AttnLayout &lay, BlockScratch &scr, RopeCache &rope, KernelTimer *t, int precision,
                       XBound *xb) {
    if (!scr.ensure(d, tokens)) return false;
    const float *rt = nullptr;
    if (!rope.get_interleaved(lay.L, d.dim_head, s, &rt)) return false;
    const int D = d.dim, inner = d.inner(), nq = d.qkvg_dim();
    float *normed = scr.normed.f(), *qkvg = scr.qkvg.f(), *attn = scr.attn.f(), *hid = scr.hidden.f();
    const int gate = d.gated ? d.qkv_dim() : -1;
    const int ff1_epi = d.ffn_glu ? EPI_GEGLU : EPI_GELU;
    if (precision == PREC_BF16) {
        // bf16 variant: the normalised activations, the fused projection, the
        // attention output and the FFN hidden layer are stored as bf16 -- the
        // operands the matrix cores take -- and the residual stream stays fp32.
        if (!(w.wqkvg_h && w.wout_h && w.w1_h && w.w2_h)) {
            set_error("transformer: bf16 weights not prepared");
            return false;
        }
        auto lin = [&](const void *A, int lda, const void *Wh, const float *bias, void *C, int ldc, int N, int K,
                       int epi, bool c16, const char *name) {
            GemmArgsBF16 g{A, lda, Wh, bf16_pitch(K), bias, C, ldc, tokens, N, K};
            g.a_bf16 = true;
            g.c_bf16 = c16;
            return gemm_bf16(s, g, epi, t, name);
        };
        if (!rmsnorm_bf16(s, x, D, w.gamma, normed, D, tokens, D, t)) return false;
        if (!lin(normed, D, w.wqkvg_h, w.bqkvg, qkvg, nq, nq, D, EPI_STORE, true, "gemm_qkv")) return false;
        if (!attention(s, qkvg, nq, attn, inner, rt, lay, d.heads, gate, t, true, true)) return false;
        if (!lin(attn, inner, w.wout_h, nullptr, x, D, D, inner, EPI_RESIDUAL, false, "gemm_out")) return false;
        if (!rmsnorm_bf16(s, x, D, w.ff_gamma, normed, D, tokens, D, t)) return false;
        if (!lin(normed, D, w.w1_h, w.b1, hid, d.ff_dim, d.ff1_out(), D, ff1_epi, true, "gemm_ff1")) return false;
        return lin(hid, d.ff_dim, w.w2_h, w.b2, x, D, D, d.ff_dim, EPI_RESIDUAL, false, "gemm_ff2");
    }
    // fp32 linears: fp16 two-piece planes on the matrix cores (A bounded by
    // bounds[slot]; a_h2: A arrives split by its producer), or the fp32 MFMA GEMM
    auto use_h2 = [&](const void *Wp, int K) {
        return Wp && w.bounds && precision == PREC_FP32 && K % SPLIT_K_MULTIPLE == 0;
    };
    auto lin = [&](const float *A, int lda, const float *W, const void *Wp, int slot, const float *bias, float *C,
                   int ldc, int N, int K, int epi, bool a_h2, const char *name) {
        if (use_h2(Wp, K)) {
            GemmArgsH2 g{A, lda, Wp, bias, C, ldc, tokens, N, K};
            g.a_h2 = a_h2;
            return gemm_h2(s, g, OperandBound{w.bounds + slot, 0.0f}, epi, t, name);
        }
        return gemm(s, {A, lda, W, K, bias, C, ldc, tokens, N, K}, epi, t, name);
    };
    const bool qkv_h2 = use_h2(w.wqkvg_p, D);
    const bool ff1_h2 = use_h2(w.w1_p, D);
    const bool att_h2 = precision == PREC_FP32 && w.bounds && w.att_h2;
    if (xb && xb->dev && xb->scratch && qkv_h2 && ff1_h2 && w.wqkvg_pg && use_h2(w.wout_p, inner) &&
        use_h2(w.w2_p, d.ff_dim)) {
        // The attention's pre-norm inside the QKV GEMM (row_norm, the gain in
        // its pieces), A = x bounded by max |x| in xb->dev: found by an
        // absmax pass or raised by the previous block's FFN down-projection
        // epilogue.  The FFN-up GEMM (after the QKV GEMM's last read of the
        // slot) zeroes it for this block's FFN down-projection to raise.  The
        // FFN's pre-norm stays a pass of its own: inside the FFN-up GEMM the
        // split of A, repeated in each of its 24 column tiles, cost more
        // (+9%) than the pass it saves.
        if (!xb->valid && !absmax(s, x, tokens * D, xb->scratch, xb->dev)) return false;
        xb->valid = false;  // until the FFN down-projection has raised the slot
        GemmArgsH2 gq{x, D, w.wqkvg_pg, w.bqkvg, qkvg, nq, tokens, nq, D};
        gq.row_norm = true;
        // k and v written times the attention's piece scales, so its staging
        // splits them without a multiply (the same bits: VOCALARC_KV_PRESCALE=0
        // keeps them unscaled, to check that)
        const char *kv_env = getenv("VOCALARC_KV_PRESCALE");
        const bool kv_pre = att_h2 && inner % 32 == 0 && !(kv_env && kv_env[0] == '0');
        if (kv_pre) {
            gq.kv_bound = w.bounds + 1;
            gq.kv_inner = inner;
        }
        // On the time axis of the [chunk][frame][band] token order, k (rotated)
        // and v leave the QKV GEMM as the attention's fp16 pieces, which it
        // copies into LDS without computing (attention_h2_kvp_kernel): the
        // rotation and the split happen once per element instead of once per
        // query group.  VOCALARC_KV_PIECES=0 keeps them fp32 (the same bits).
        const char *kvp_env = getenv("VOCALARC_KV_PIECES");
        const bool kv_pieces = kv_pre && lay.L > 64 && inner % 128 == 0 && lay.seq_stride == 1 &&
                               lay.pos_stride == lay.group && lay.group_stride == lay.group * lay.L &&
                               !(kvp_env && kvp_env[0] == '0');
        if (kv_pieces) {
            gq.kv_pieces = true;
            gq.rope = rt;
            gq.rope_period = lay.group;
            gq.rope_len = lay.L;
        }
        // On the band axis (sequences of L <= 64 consecutive rows) the
        // projection and the attention run as one kernel (band_attention.hpp):
        // q, k, v and the gate logits stay on chip.  VOCALARC_BAND_FUSED=0
        // keeps the two kernels.
        const char *bf_env = getenv("VOCALARC_BAND_FUSED");
        const bool band_fused = kv_pre && lay.L <= 64 && lay.group == 1 && lay.seq_stride == 0 &&
                                lay.pos_stride == 1 && lay.group_stride == lay.L && tokens == (int64_t)lay.S * lay.L &&
                                D <= BA_MAX_K && inner % GS_BN == 0 && (!d.gated || w.wgate_g) && rt &&
                                !(bf_env && bf_env[0] == '0');
        if (band_fused) {
            BandAttention ba{x, D, D, w.wqkvg_pg, w.bqkvg, d.gated ? w.wgate_g : nullptr,
                             d.gated && w.bqkvg ? w.bqkvg + d.qkv_dim() : nullptr, xb->dev, w.bounds + 1, rt,
                             attn, inner, lay.S, lay.L, d.heads};
            if (!band_attention(s, ba, t)) return false;
        } else {
            if (!gemm_h2(s, gq, OperandBound{xb->dev, 0.0f}, EPI_STORE, t, "gemm_qkv")) return false;
            if (!attention(s, qkvg, nq, attn, inner, rt, lay, d.heads, gate, t, false, false, true,
                           att_h2 ? w.bounds + 1 : nullptr, att_h2, kv_pre, false, kv_pieces))
                return false;
        }
        if (!lin(attn, inner, w.wout, w.wout_p, 1, nullptr, x, D, D, inner, EPI_RESIDUAL, att_h2, "gemm_out"))
            return false;
        if (!rmsnorm_h2(s, x, D, w.ff_gamma, normed, D, tokens, D, w.bounds + 2, t)) return false;
        GemmArgsH2 g1{normed, D, w.w1_p, w.b1, hid, d.ff_dim, tokens, d.ff1_out(), D};
        g1.a_h2 = true;
        g1.zero_slot = xb->dev;
        if (!gemm_h2(s, g1, OperandBound{w.bounds + 2, 0.0f}, ff1_epi, t, "gemm_ff1")) return false;
        GemmArgsH2 g2{hid, d.ff_dim, w.w2_p, w.b2, x, D, tokens, D, d.ff_dim};
        g2.amax = xb->dev;
        if (!gemm_h2(s, g2, OperandBound{w.bounds + 3, 0.0f}, EPI_RESIDUAL, t, "gemm_ff2")) return false;
        xb->valid = true;
        return true;
    }
    if (xb) xb->valid = false;
    // pre-norm (split into fp16 pieces for the two-piece GEMM) -> fused QKV
    // (+gate logits with their bias)
    if (!(qkv_h2 ? rmsnorm_h2(s, x, D, w.gamma, normed, D, tokens, D, w.bounds, t)
                 : rmsnorm(s, x, D, w.gamma, normed, D, tokens, D, t)))
        return false;
    if (!lin(normed, D, w.wqkvg, w.wqkvg_p, 0, w.bqkvg, qkvg, nq, nq, D, EPI_STORE, qkv_h2, "gemm_qkv")) return false;
    // rotary + attention + gates (products as fp16 two-piece splits on the
    // default fp32 path)
    // the two-piece attention writes its output as the out projection's
    // pieces when that GEMM runs on them (same bound: the value bound)
    const bool attn_rows = att_h2 && use_h2(w.wout_p, inner);
    if (!attention(s, qkvg, nq, attn, inner, rt, lay, d.heads, gate, t, false, false, precision == PREC_FP32,
                   att_h2 ? w.bounds + 1 : nullptr, attn_rows))
        return false;
    // out projection added to the residual stream
    if (!lin(attn, inner, w.wout, w.wout_p, 1, nullptr, x, D, D, inner, EPI_RESIDUAL, attn_rows, "gemm_out"))
        return false;
    // FFN
    if (!(ff1_h2 ? rmsnorm_h2(s, x, D, w.ff_gamma, normed, D, tokens, D, w.bounds + 2, t)
                 : rmsnorm(s, x, D, w.ff_gamma, normed, D, tokens, D, t)))
        return false;
    if (!lin(normed, D, w.w1, w.w1_p, 2, w.b1, hid, d.ff_dim, d.ff1_out(), D, ff1_epi, ff1_h2, "gemm_ff1")) return false;
    return lin(hid, d.ff_dim, w.w2, w.w2_p, 3, w.b2, x, D, D, d.ff_dim, EPI_RESIDUAL, false, "gemm_ff2");
}

// ---------------------------------------------------------------- upload
bool upload_weight(hipStream_t s, const float *host_packed, int in, int out, float *dst, int ldd, int row0, int mode,
                   DeviceBuffer &staging) {
    const size_t bytes = (size_t)in * out * sizeof(float);
    if (!staging.ensure(bytes, "hipMalloc(weight staging)")) return false;
    if (!check(hipMemcpyAsync(staging.ptr, host_packed, bytes, hipMemcpyHostToDevice, s), "hipMemcpy(weight)"))
        return false;
    if (!unpack_weight(s, staging.f(), in, out, dst, ldd, row0, mode)) return false;
    // The staging buffer is reused by the next upload: wait for the unpack.
    return check(hipStreamSynchronize(s), "hipStreamSynchronize(weight)");
}

bool upload_vector(hipStream_t s, const float *host, size_t count, float *dst) {
    if (!check(hipMemcpyAsync(dst, host, count * sizeof(float), hipMemcpyHostToDevice, s), "hipMemcpy(vector)"))
        return false;
    return check(hipStreamSynchronize(s), "hipStreamSynchronize(vector)");
}

}  // namespace vh
