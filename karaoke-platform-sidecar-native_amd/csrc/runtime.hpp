// Host-side runtime of the VocalArc HIP provider: device buffers, the
// per-shape launchers of the gfx950 kernels, weight upload and the
// device-resident transformer block shared by the native_gpu.h provider and
// the vocalarc_hip.h harness API.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/vocalarc_hip.h"

namespace vh {

// ----------------------------------------------------------------- errors
// Every HIP call goes through check(); the first failure is remembered (for
// vh_last_error) and printed once with the operation name.
bool check(hipError_t e, const char *what);
void set_error(const char *fmt, ...);
const char *last_error();
bool debug_enabled();
bool sync_debug(hipStream_t s, const char *what);

// ---------------------------------------------------------------- buffers
struct DeviceBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
    bool ensure(size_t need, const char *what);
    void release();
    float *f() const { return static_cast<float *>(ptr); }
    ~DeviceBuffer() { release(); }
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
};

// --------------------------------------------------------------- kernel timing
// Optional per-kernel-class timing with HIP events recorded on the launch
// stream around each launch of a named class (e.g. "gemm_ff1").
struct KernelTimer {
    bool enabled = false;
    bool all = false;
    std::vector<std::string> only;  // classes to time when !all
    bool wants(const char *name) const;
    struct Pending { std::string name; hipEvent_t a, b; };
    std::vector<Pending> pending;
    std::map<std::string, std::pair<double, int64_t>> totals;  // ms, count
    void begin(hipStream_t s, const char *name, hipEvent_t *a);
    void end(hipStream_t s, const char *name, hipEvent_t a);
    void collect();  // after a stream sync
    void reset();
};

struct Scope {
    KernelTimer *t;
    hipStream_t s;
    const char *name;
    hipEvent_t a = nullptr;
    Scope(KernelTimer *t_, hipStream_t s_, const char *n) : t(t_), s(s_), name(n) {
        if (t && t->enabled && t->wants(name)) t->begin(s, name, &a);
    }
    ~Scope() {
        if (a) t->end(s, name, a);
    }
};

// --------------------------------------------------------------- launchers
// GEMM epilogues (what the store does with acc + bias).
enum Epilogue : int {
    EPI_STORE = 0,     // C = acc + bias
    EPI_GELU = 1,      // C = gelu(acc + bias)
    EPI_TANH = 2,      // C = tanh(acc + bias)
    EPI_RESIDUAL = 3,  // C += acc + bias
    EPI_GEGLU = 4,     // columns come in (32 value, 32 gate) pairs: C[:, n/2] = v * gelu(g)
};

struct GemmArgs {
    const float *A; int lda;
    const float *B; int ldb;  // [N][K] rows
    const float *bias;
    float *C; int ldc;
    int64_t M; int N, K;
};
bool gemm(hipStream_t s, const GemmArgs &g, int epilogue, KernelTimer *t = nullptr, const char *name = "gemm");
// Batched/ragged: one descriptor per problem, launched together.
bool gemm_batched(hipStream_t s, const std::vector<GemmArgs> &g, int epilogue, KernelTimer *t = nullptr,
                  const char *name = "gemm_batched");

// bf16-MFMA variant: A fp32 (rounded to bf16 on the way into LDS), B a bf16
// weight copy with row pitch ldb >= K rounded up to 8 and zero padding.
struct GemmArgsBF16 {
    const void *A; int lda;  // fp32, or bf16 when a_bf16 (then K and lda multiples of 8)
    const void *B; int ldb;  // bf16 [N][ldb]
    const float *bias;
    void *C; int ldc;        // fp32, or bf16 when c_bf16 (not with the residual epilogue)
    int64_t M; int N, K;
    bool a_bf16 = false, c_bf16 = false;
    bool staged = false;     // bf16 A with K % 32 == 0: force the register-staged kernel over the DMA ring
};
bool gemm_bf16(hipStream_t s, const GemmArgsBF16 &g, int epilogue, KernelTimer *t = nullptr,
               const char *name = "gemm_bf16");
bool gemm_bf16_batched(hipStream_t s, const std::vector<GemmArgsBF16> &g, int epilogue, KernelTimer *t = nullptr,
                       const char *name = "gemm_bf16_batched");
// fp32-accurate linear on bf16 matrix cores (gemm_split.hpp): A fp32, W as
// its three bf16 pieces in the tile-major layout split_weights writes, C fp32.
// K a multiple of 16; lda a multiple of 4; A and W 16-byte aligned.
struct GemmArgsSplit {
    const float *A; int lda;
    const void *W;
    const float *bias;
    float *C; int ldc;
    int64_t M; int N, K;
};
bool gemm_split(hipStream_t s, const GemmArgsSplit &g, int epilogue, KernelTimer *t = nullptr,
                const char *name = "gemm_split");
// K granularity of gemm_split, and the bytes of W's pieces (N rounded up to
// a multiple of 128).
constexpr int SPLIT_K_MULTIPLE = 16;
inline size_t split_bytes(int N, int K) { return (size_t)(N + 127) / 128 * 128 * K * 6; }
// fp32 W [N][ldw] -> its h, m, l bf16 pieces (h = bf16(w), m = bf16(w - h),
// l = w - h - m), tile-major for gemm_split (split_bytes(N, K) bytes).
bool split_weights(hipStream_t s, const float *W, int N, int K, int ldw, void *pieces);

// fp32-accurate linear on fp16 matrix cores (gemm_h2.hpp): A fp32 with every
// |A| element at most the bound, W as its two fp16 pieces (split_weights_h2),
// C fp32.  K a multiple of 16; lda a multiple of 4 and at most 2^21; A 16-byte
// aligned.  The bound is a device float (dev) or a value.
struct GemmArgsH2 {
    const float *A; int lda;
    const void *W;
    const float *bias;
    float *C; int ldc;
    int64_t M; int N, K;
    bool a_h2 = false;  // A given as h2 rows (h2.hpp) scaled from the same bound
    // fp32 A rows RMSNorm-ed inside the GEMM, W holding the gain (gemm_h2_body
    // NORM): each output row times sqrt(K) / sqrt(sum_k A^2 + 1e-12) before
    // bias and activation (EPI_STORE, EPI_GELU, EPI_GEGLU)
    bool row_norm = false;
    float *zero_slot = nullptr;  // a device float the kernel sets to 0
    float *amax = nullptr;       // EPI_RESIDUAL: raised to max |C| written
    // kv_inner > 0 (a multiple of 32; EPI_STORE with row_norm): C is a fused
    // q|k|v|gates projection whose k and v columns are written times 2^ek and
    // 2^ev of the attention bound *kv_bound (GemmDescH2::kv_inner)
    const float *kv_bound = nullptr;
    int kv_inner = 0;
    // with kv_inner (a multiple of 128): k (rotated by the interleaved table
    // rope of rope_len positions, row r at frame (r / rope_period) % rope_len)
    // and v written as fp16 pieces for attention(kv_pieces) (GemmDescH2)
    bool kv_pieces = false;
    const float *rope = nullptr;
    int rope_period = 0, rope_len = 0;
};
struct OperandBound {
    const float *dev = nullptr;
    float value = 0.0f;
};
bool gemm_h2(hipStream_t s, const GemmArgsH2 &g, const OperandBound &bound, int epilogue, KernelTimer *t = nullptr,
             const char *name = "gemm_h2");
// A ragged batch of fp16 two-piece GEMMs with one A bound (one launch per 64 problems).
bool gemm_h2_batched(hipStream_t s, const std::vector<GemmArgsH2> &gs, const OperandBound &bound, int epilogue,
                     KernelTimer *t = nullptr, const char *name = "gemm_h2");
// The band-axis attention fused with its pre-norm projection
// (band_attention.hpp): for S sequences of L <= 64 consecutive rows of the
// residual stream x, the q, k, v and gate columns of the gain-folded fused
// projection (W: its pieces, rows q|k|v of heads * 64 each, then the gates;
// gate_w: the gate rows in fp32 with the gain folded, null for none), the
// rotary attention with the fp16 two-piece products, and out written as h2
// rows scaled by 2^h2_exponent(*bound) (the out projection's A).  x_bound:
// max |x| (device float); bound: the fused projection's bound (device float,
// within the two-piece attention's range); rope: the interleaved rotary table
// of at least L positions (required).  K a multiple of 16 and at most
// 512; heads * 64 a multiple of 128; out must not overlap x.
struct BandAttention {
    const float *x; int lda, K;
    const void *W;
    const float *bias;
    const float *gate_w, *gate_b;
    const float *x_bound, *bound, *rope;
    float *out; int ld_out;
    int S, L, heads;
};
bool band_attention(hipStream_t s, const BandAttention &b, KernelTimer *t = nullptr);
// Bytes of W's fp16 pieces: a 256-byte header (max|W|) and two planes (N
// rounded up to a multiple of 128).
inline size_t h2_bytes(int N, int K) { return 256 + (size_t)(N + 127) / 128 * 128 * K * 4; }
// fp32 W [N][ldw] -> max|W| and the h, m fp16 pieces of W * 2^e
// (h2_bytes(N, K) bytes, 256-byte aligned).
bool split_weights_h2(hipStream_t s, const float *W, int N, int K, int ldw, void *pieces);
// The same for W with column k multiplied by gamma[k] (an RMSNorm gain folded
// into the matrix after it, for gemm_h2 row_norm); tmp: N*K device floats.
bool fold_gain_split_h2(hipStream_t s, const float *W, int N, int K, int ldw, const float *gamma, float *tmp,
                        void *pieces);
// Device bounds for the fp16 two-piece GEMM's A operands downstream of an
// RMSNorm with gain gamma[D] (operand_bounds_kernel in gemm_h2.hpp):
// out[0] bounds the normalised activations, out[1] (when W [N][D] is given)
// every output of W y + b, or its square when `square` (a GELU-GLU of two).
bool operand_bounds(hipStream_t s, const float *gamma, int D, const float *W, int N, const float *b, bool square,
                    float *out);

// max |x[i]| over n floats into the device float out (scratch: ABSMAX_PARTIALS
// device floats).
constexpr int ABSMAX_PARTIALS = 1024;
bool absmax(hipStream_t s, const float *x, int64_t n, float *scratch, float *out);

// fp32 [rows][cols] -> bf16 [rows][ld] (ld >= cols, padding zeroed by the caller)
bool to_bf16_rows(hipStream_t s, const float *src, int rows, int cols, void *dst, int ld);
inline int bf16_pitch(int k) { return (k + 7) & ~7; }

bool rmsnorm(hipStream_t s, const float *x, int ldx, const float *gamma, float *y, int ldy, int64_t rows, int dim,
             KernelTimer *t = nullptr);
// Same, bf16 output (y is bf16 [rows][ldy]).
bool rmsnorm_bf16(hipStream_t s, const float *x, int ldx, const float *gamma, void *y, int ldy, int64_t rows, int dim,
                  KernelTimer *t = nullptr);
// Same, y written as h2 rows (h2.hpp) scaled by 2^h2_exponent(*bound) for a
// fp16 two-piece GEMM with a_h2 (dim a multiple of 16).
bool rmsnorm_h2(hipStream_t s, const float *x, int ldx, const float *gamma, float *y, int ldy, int64_t rows, int dim,
                const float *bound, KernelTimer *t = nullptr);
bool softmax_rows(hipStream_t s, const float *in, float *out, int64_t rows, int len, KernelTimer *t = nullptr);
bool rope_bhld(hipStream_t s, float *x, const float *cs, const float *sn, int64_t bh, int len,
               KernelTimer *t = nullptr);
bool geglu(hipStream_t s, const float *in, float *out, int64_t rows, int width, KernelTimer *t = nullptr);
bool residual_add(hipStream_t s, float *x, const float *r, int64_t n, KernelTimer *t = nullptr);
bool unpack_weight(hipStream_t s, const float *packed_dev, int in, int out, float *dst, int ldd, int row0,
                   int mode);
bool interleave_glu_bias(hipStream_t s, const float *src, float *dst, int out);
bool transpose_rows(hipStream_t s, const float *src, float *dst, int outer, int a, int b, int dim);

struct AttnLayout {
    int S, L;
    int group, group_stride, seq_stride, pos_stride;
};
// qkv fp32 (fp32 MFMA) or, with qkv_bf16, bf16 (bf16 MFMA); out fp32, or bf16
// when out_bf16.  split (fp32 qkv): the products in fp32 accuracy on the
// matrix cores -- as two-piece fp16 splits when `bound` (a device float
// bounding |q|, |k|, |v|) is given (attention_h2.hpp, any L), else, for
// L > 64, as exact three-piece bf16 splits (attention_split.hpp; L <= 64
// keeps the fp32 MFMA kernel).  rope: interleaved rotary
// table of length lay.L (or null).  out_h2 (with `bound`): out written as h2
// rows scaled by 2^h2_exponent(*bound), for a gemm_h2 with a_h2 and that bound.
// kv_scaled (with `bound`, fp32 qkv and out): the k and v columns arrive
// times 2^ek and 2^ev, as a gemm_h2 with kv_inner and that bound writes them.
// device_choice (with split and `bound`, neither out_h2 nor kv_scaled): the
// bound may lie outside the two-piece kernels' scale range and is not read
// back -- the two-piece kernel and the kernel without piece scales are both
// launched, each returning at once unless the bound's range selects it
// (AttnArgs::guard), so the call never synchronises.
// kv_pieces (with kv_scaled, L > 64): k and v arrive as the fp16 pieces a
// gemm_h2 with kv_pieces writes (k rotated; rope must be the table it used).
bool attention(hipStream_t s, const void *qkv, int ld, void *out, int ld_out, const float *rope, const AttnLayout &lay,
               int heads, int gate_col, KernelTimer *t = nullptr, bool out_bf16 = false, bool qkv_bf16 = false,
               bool split = false, const float *bound = nullptr, bool out_h2 = false, bool kv_scaled = false,
               bool device_choice = false, bool kv_pieces = false);

// ------------------------------------------------------------------- dims
struct Dims {
    int dim, depth, bands, heads, dim_head, ff_dim, ffn_glu, gated, mask_hidden, n_fft, hop, channels;
    int band_widths[VH_MAX_BANDS];
    int freq_bins() const { return n_fft / 2 + 1; }
    int inner() const { return heads * dim_head; }
    int qkv_dim() const { return 3 * inner(); }
    int ff1_out() const { return ffn_glu ? 2 * ff_dim : ff_dim; }
    // fused QKV + gate projection width (gates padded to a 32-column tile)
    int qkvg_dim() const { return qkv_dim() + (gated ? 32 : 0); }
    int in_dim(int b) const { return band_widths[b] * channels * 2; }
    int frames(int length) const { return length / hop + 1; }
    bool valid(char *why, size_t n) const;
};
Dims dims_from(const vh_dims &d);

// ------------------------------------------------------- device weights
struct LayerWeights {
    float *gamma = nullptr, *ff_gamma = nullptr;
    float *wqkvg = nullptr, *bqkvg = nullptr;  // [qkvg_dim][D], bias (0 on q/k/v columns)
    float *wout = nullptr;                     // [D][inner]
    float *w1 = nullptr, *b1 = nullptr;        // [ff1_out][D] (value/gate interleaved for GLU)
    float *w2 = nullptr, *b2 = nullptr;        // [D][ff_dim]
    // bf16 copies for the reduced-precision variant (null: fp32 only)
    void *wqkvg_h = nullptr, *wout_h = nullptr, *w1_h = nullptr, *w2_h = nullptr;
    // fp16 two-piece planes (split_weights_h2) for the fp32 path on fp16
    // matrix cores, and the device bounds of their A operands {QKV, out,
    // FFN up, FFN down} (layer_bounds); null: the fp32 MFMA GEMM runs instead
    void *wqkvg_p = nullptr, *wout_p = nullptr, *w1_p = nullptr, *w2_p = nullptr;
    // the same pieces of the QKV matrix with its RMSNorm gain folded in
    // (fold_gain_split_h2), for blocks whose attention pre-norm runs inside
    // that GEMM (XBound); null: the RMSNorm kernel runs
    void *wqkvg_pg = nullptr;
    // the gate rows of that gain-folded matrix in fp32 ([heads][D]), for the
    // band-axis attention fused with its projection; null: not fused
    float *wgate_g = nullptr;
    float *bounds = nullptr;
    // the fused projection's bound (bounds[1], which also bounds q, k and v)
    // lies in the fp16 two-piece attention's range (h2_attention_bound_ok);
    // false: the attention runs on the kernels without piece scales
    bool att_h2 = false;
};
// The four A-operand bounds of a layer's linears into the device floats
// bounds[0..3] (operand_bounds on its two RMSNorm gains and the matrices they
// feed; bounds[1], on the fused projection's q, k, v rows, also bounds the
// attention output).
bool layer_bounds(hipStream_t s, const Dims &d, const LayerWeights &w, float *bounds);
// Reads n (<= 8) device bounds back (into host[0..n) when host is not
// null): 1 when all are finite and within the fp16 two-piece GEMM's scale
// range (<= 1e30), 0 when not (those products then run on the fp32 MFMA
// instruction), -1 on a runtime error.  Synchronous.
int bounds_usable(hipStream_t s, const float *dev, int n, float *host = nullptr);

// Arithmetic of the matrix products.  PREC_FP32 (the parity path): fp32
// accuracy, the transformer linears on fp16 matrix cores by two-piece operand
// splitting where the planes exist, the fp32 MFMA GEMM elsewhere.
// PREC_FP32_MFMA: every product on the fp32 MFMA instruction.  PREC_BF16:
// bf16 operands with fp32 accumulation (separately reported variant).
enum Precision : int { PREC_FP32 = 0, PREC_BF16 = 1, PREC_FP32_MFMA = 2 };

// The rotary tables of positions 0..length-1 with base 10000, built on the
// host with the reference's float expressions (native/vocalarc_separation.c:
// 726-731,1312) so they are bit-exact: cos_t/sin_t [length][dim_head/2] and
// the same values interleaved as (cos, sin) pairs [length][dim_head/2][2], so
// one 16-byte load gives what four rotated dims need; null outputs are
// skipped.  An entry depends only on its position and pair, so the table of
// a length is a prefix of every longer one's.
void rope_table_host(int length, int dim_head, float *cos_t, float *sin_t, float *interleaved);

struct RopeCache {
    struct Tables { float *cos, *sin, *interleaved; };
    std::map<int, Tables> tables;
    bool get(int length, int dim_head, hipStream_t s, const float **cs, const float **sn);
    bool get_interleaved(int length, int dim_head, hipStream_t s, const float **cssn);
    void release();
    ~RopeCache() { release(); }
};

// Scratch for one transformer pass over `tokens` tokens.
struct BlockScratch {
    DeviceBuffer normed, qkvg, attn, hidden;
    bool ensure(const Dims &d, int64_t tokens);
};

// One axial transformer block on device-resident activations x
// (native/vocalarc_separation.c:836-873).  Rows of x are tokens; `lay` maps
// (sequence, position) to rows.
// Bound slot of the residual stream x for blocks whose attention pre-norm runs
// inside the QKV GEMM (gemm_h2 row_norm; its fp32 A is x itself, split by the
// bound of |x|): *dev bounds x entering a block -- raised by the previous
// block's FFN-down epilogue, which `valid` records, else found by an absmax
// pass.  scratch: ABSMAX_PARTIALS device floats.
struct XBound {
    float *dev = nullptr;
    float *scratch = nullptr;
    bool valid = false;
};
// One pre-norm transformer block on x in place.  With xb (and the gain-folded
// QKV pieces in w, every linear on the fp16 pieces) the attention's pre-norm
// is fused into the QKV GEMM; otherwise the RMSNorm kernel writes the
// normalised rows for both.
bool transformer_block(hipStream_t s, const Dims &d, const LayerWeights &w, float *x, int64_t tokens,
                       const AttnLayout &lay, BlockScratch &scr, RopeCache &rope, KernelTimer *t = nullptr,
                       int precision = PREC_FP32, XBound *xb = nullptr);

// Host packed weight (reference layout) -> device [out][in] rows, through a
// staging buffer.  mode as unpack_weight.
bool upload_weight(hipStream_t s, const float *host_packed, int in, int out, float *dst, int ldd, int row0, int mode,
                   DeviceBuffer &staging);
bool upload_vector(hipStream_t s, const float *host, size_t count, float *dst);

}  // namespace vh
