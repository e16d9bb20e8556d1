// The C-ABI of libnncpu_hip.so (include/nncpu_hip.h): weight upload, the
// model_gemv / gemv_batch / model_argmax dispatch on the uploaded weight's
// format (crates/nncpu/src/model/mod.rs:417-444, model/forward.rs:15-58,
// 989-1011), and the device-resident entry points.
//
// One process-wide context (device, one non-blocking stream at default
// priority, a device scratch buffer per calling stream and pinned staging)
// guarded by a mutex, as the reference's pool serialises dispatch
// (pool.rs:7-9,253).
//
// Device memory per weight: nncpu's split layout as uploaded, plus derived
// layouts built on the first call that reads them (each one once, under the
// mutex, synchronised), so a weight used in one mode holds only that mode's
// copies.

#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "f32_m1.h"
#include "nncpu_hip.h"

struct nnh_weight {
    int dtype;
    int device;
    size_t rows, cols, nb, nbp;
    uint8_t* raw;         // device: nncpu's split layout, as uploaded
    const uint8_t* qs;    // views into raw
    const uint16_t* sc;
    const uint16_t* bi;   // Q4 only
    uint32_t* sb;         // device: Q4 scale | bias << 16 per block (int8 path)
    uint8_t* fq;          // device: per-lane quant groups for the f32 path
    bool f32v2;           // fq in the 8-lane layout (tall matrices)
    uint16_t* fs;         // device: scales padded to nbp per row
    float* swT;           // device: [nb][rows padded] f32 scales, Q4 biases after (MFMA GEMM)
    int bpath;            // BF16 only: the reference kernel this shape takes (nnh::BF16_PATH_*)
    uint16_t* bl;         // device: BF16 only, the chain layout (none on the f64 path)
    uint16_t* wbi;        // device: Q4 biases twice per block, rows padded (MX GEMM)
    unsigned ready;       // derived layouts built so far (LAY_* bits)
    size_t dev_bytes;     // device bytes held (split layout + derived layouts)
};

namespace {

thread_local std::string t_err;
std::mutex g_mu;
int g_device = -1;
hipStream_t g_stream = nullptr;
// Device scratch per calling stream (the host-buffer calls use g_stream's),
// so calls on different streams never share one. A buffer that grows is
// retired, not freed: a HIP graph that captured a call keeps its address.
// nnh_stream_release frees a stream's buffers, retired ones included.
struct Scratch {
    uint8_t* p = nullptr;
    size_t bytes = 0;
    std::vector<uint8_t*> retired;  // outgrown buffers, freed by nnh_stream_release
};
std::unordered_map<hipStream_t, Scratch> g_scratch;
uint8_t* g_pinned = nullptr;  // pinned host staging for the host-buffer calls
size_t g_pinned_bytes = 0;

// The scratch of nnh_gemv_batch_dev_noalloc, for callers that cannot
// allocate: a device array each GPU holds for the process's lifetime, at its
// own address, looked up once per device at init (g_noalloc). Host code
// never passes the array's name to a kernel or copy: in host code it is a
// stand-in, not a device address.
static __device__ __align__(256) uint8_t scratch[NNH_NOALLOC_SCRATCH_BYTES];
uint8_t* g_noalloc = nullptr;  // device address of `scratch` on g_device

int fail(int code, const std::string& msg) {
    t_err = msg;
    return code;
}

#define NNH_HIP(expr)                                                                              \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess)                                                                      \
            return fail(e_ == hipErrorOutOfMemory ? NNH_E_OOM : NNH_E_DEVICE,                      \
                        std::string(#expr) + ": " + hipGetErrorString(e_));                        \
    } while (0)

constexpr size_t ALIGN = 256;
inline size_t align_up(size_t v) { return (v + ALIGN - 1) / ALIGN * ALIGN; }

// Caller holds g_mu.
int init_locked(int device) {
    if (g_device >= 0) {
        if (device != g_device) return fail(NNH_E_STATE, "nnh_init: already initialised on another device");
        NNH_HIP(hipSetDevice(g_device));
        return NNH_OK;
    }
    int count = 0;
    NNH_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return fail(NNH_E_STATE, "nnh_init: no such device");
    NNH_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    NNH_HIP(hipGetDeviceProperties(&prop, device));
    if (std::string(prop.gcnArchName).find("gfx950") == std::string::npos)
        return fail(NNH_E_STATE, std::string("nnh_init: built for gfx950, device is ") + prop.gcnArchName);
    void* na = nullptr;
    NNH_HIP(hipGetSymbolAddress(&na, HIP_SYMBOL(scratch)));
    if (!na) return fail(NNH_E_DEVICE, "nnh_init: no device address for the no-alloc scratch");
    NNH_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    g_noalloc = (uint8_t*)na;
    g_device = device;
    return NNH_OK;
}

int ensure_locked() { return init_locked(g_device >= 0 ? g_device : 0); }

// The scratch of calls on `st`, at least `bytes`; caller holds g_mu. Work
// queued on `st` (or replays of graphs captured on it) may still use the
// old buffer, so a grown buffer keeps the old one alive until
// nnh_stream_release (or the process end); doubling bounds the retired
// total by the live size.
int scratch_locked(hipStream_t st, size_t bytes, uint8_t** out) {
    Scratch& s = g_scratch[st];
    if (bytes > s.bytes) {
        const size_t want = align_up(bytes > 2 * s.bytes ? bytes : 2 * s.bytes);
        uint8_t* p = nullptr;
        NNH_HIP(hipMalloc((void**)&p, want));
        if (s.p) s.retired.push_back(s.p);
        s.p = p;
        s.bytes = want;
    }
    *out = s.p;
    return NNH_OK;
}

// Grow the pinned host staging buffer to `bytes`; caller holds g_mu and no
// queued work reads the old one (every host-buffer call ends synchronised).
int pinned_locked(size_t bytes, uint8_t** out) {
    if (bytes > g_pinned_bytes) {
        if (g_pinned) {
            NNH_HIP(hipHostFree(g_pinned));
            g_pinned = nullptr;
            g_pinned_bytes = 0;
        }
        size_t want = align_up(bytes + bytes / 4);
        NNH_HIP(hipHostMalloc((void**)&g_pinned, want, hipHostMallocDefault));
        g_pinned_bytes = want;
    }
    *out = g_pinned;
    return NNH_OK;
}

struct ActLayout {
    size_t off_s, off_sx, off_sxT, off_xb, off_xl, bytes;
};

// q[n_tok][cols] i8, s[n_tok][nb] bf16, sx[n_tok][nb][2] f64, then the
// GEMM's block-major copies sxT[2][nb][tok_pad] f32; MX adds the BF16
// operands of its GEMM, xb[n_tok][cols] and xl[tok_pad][nbp8][2].
ActLayout act_layout(size_t cols, size_t n_tok, int act = NNH_ACT_I8) {
    size_t nb = cols / 32;
    ActLayout l;
    l.off_s = align_up(n_tok * cols);
    l.off_sx = l.off_s + align_up(n_tok * nb * 2);
    l.off_sxT = l.off_sx + align_up(n_tok * nb * 16);
    l.off_xb = l.off_sxT + align_up(2 * nb * (size_t)nnh::gemm_tok_pad((int)n_tok) * 4);
    l.off_xl = l.off_xb;
    l.bytes = l.off_xb;
    if (act == NNH_ACT_MXI8) {
        l.off_xl = l.off_xb + align_up((size_t)nnh::mx_xl_tok((int)n_tok) * cols * 2);
        l.bytes = l.off_xl + align_up(nnh::mx_xl_bytes((int)n_tok, (int)nb));
    }
    return l;
}

void launch_quantize(int act, const float* x, size_t x_stride, size_t cols, size_t n_tok, uint8_t* a,
                     hipStream_t st) {
    const ActLayout l = act_layout(cols, n_tok, act);
    if (act == NNH_ACT_MXI8)
        nnh::launch_quantize_mx(x, x_stride, (int)cols, (int)n_tok, (int8_t*)a, (uint16_t*)(a + l.off_s),
                                (double*)(a + l.off_sx), (float*)(a + l.off_sxT), nnh::gemm_tok_pad((int)n_tok),
                                (uint16_t*)(a + l.off_xb), (uint16_t*)(a + l.off_xl), st);
    else
        nnh::launch_quantize_act(x, x_stride, (int)cols, (int)n_tok, (int8_t*)a, (uint16_t*)(a + l.off_s),
                                 (double*)(a + l.off_sx), (float*)(a + l.off_sxT), nnh::gemm_tok_pad((int)n_tok), st);
}

int check_weight(const nnh_weight* w) {
    if (!w) return fail(NNH_E_INVALID, "null weight");
    if (w->device != g_device) return fail(NNH_E_STATE, "weight belongs to another device");
    return NNH_OK;
}

// The int8 matmul on quantized activations: the sdot4 GEMV for up to 3
// vectors, the few-token MFMA kernel up to 16, the MFMA GEMM beyond
// (crossovers measured at the verify shapes: at 4 vectors the few-token
// kernel takes 6.1 / 8.5 us against the GEMV's 6.9 / 10.2).
constexpr size_t SKINNY_MIN_TOKENS = 4;
constexpr size_t GEMM_MIN_TOKENS = 17;

// Device workspace the int8 matmul needs beyond the activation buffer.
size_t i8_workspace_bytes(const nnh_weight* w, size_t n_tok, int act) {
    if (n_tok >= GEMM_MIN_TOKENS && act == NNH_ACT_MXI8)
        return nnh::gemm_mx_workspace_bytes((int)w->rows, (int)w->nb, (int)n_tok);
    if (n_tok >= GEMM_MIN_TOKENS) return nnh::gemm_workspace_bytes((int)w->rows, (int)w->nb, (int)n_tok);
    if (n_tok >= SKINNY_MIN_TOKENS) return nnh::skinny_workspace_bytes((int)w->rows, (int)w->nb);
    return 0;
}

// `mode`: NNH_ACT_I8 or NNH_ACT_MXI8, the quantizer `act` came from. Both
// buffers start with the same q / s / sx / sxT, so every kernel but the MX
// GEMM reads either.
void launch_i8(const nnh_weight* w, int mode, const uint8_t* act, size_t n_tok, float* y, size_t y_stride,
               uint8_t* ws, hipStream_t st) {
    const ActLayout l = act_layout(w->cols, n_tok, mode);
    const int8_t* q = (const int8_t*)act;
    const double* sx = (const double*)(act + l.off_sx);
    const float* sxT = (const float*)(act + l.off_sxT);
    if (n_tok >= GEMM_MIN_TOKENS && mode == NNH_ACT_MXI8)
        nnh::launch_gemm_mx(w->dtype, w->qs, w->swT, w->wbi, (const uint16_t*)(act + l.off_xb),
                            (const uint16_t*)(act + l.off_xl), (int)w->rows, (int)w->nb, (int)n_tok, y, y_stride,
                            (float*)ws, st);
    else if (n_tok >= GEMM_MIN_TOKENS)
        nnh::launch_gemm_i8(w->dtype, w->qs, w->swT, q, sxT, (int)w->rows, (int)w->nb, (int)n_tok, y, y_stride,
                            (double*)ws, st);
    else if (n_tok >= SKINNY_MIN_TOKENS)
        nnh::launch_skinny_i8(w->dtype, w->qs, w->swT, q, sxT, (int)w->rows, (int)w->nb, (int)n_tok, y, y_stride,
                              (double*)ws, st);
    else
        nnh::launch_gemv_i8(w->dtype, w->qs, w->sc, w->bi, w->sb, q, sx, (int)w->rows, (int)w->nb, (int)n_tok, y,
                            y_stride, st);
}

// Queue the matmul for device x / y; `scratch` holds xsum or the act buffer.
int run_gemv(const nnh_weight* w, const float* x, size_t x_stride, float* y, size_t y_stride, size_t n_tok, int act,
             uint8_t* scratch, hipStream_t st) {
    const int rows = (int)w->rows, nb = (int)w->nb;
    if (w->dtype == NNH_BF16) {
        nnh::launch_gemv_bf16(w->bpath, (const uint16_t*)w->raw, w->bl, rows, (int)w->cols, x, x_stride, (int)n_tok, y,
                              y_stride, st);
    } else if (act == NNH_ACT_F32) {
        float* xsum = w->dtype == NNH_Q4S ? (float*)scratch : nullptr;
        nnh::launch_gemv_f32(w->dtype, w->fq, w->fs, w->bi, x, x_stride, xsum, rows, nb, (int)w->nbp, (int)n_tok,
                             y, y_stride, w->f32v2, st);
    } else if (!(act == NNH_ACT_I8 && n_tok == 1 &&
                 nnh::launch_gemv_i8_qx(w->dtype, w->qs, w->sc, w->sb, x, rows, nb, y, st))) {
        // (One vector at most rows: quantized in the GEMV's own prologue.)
        const ActLayout l = act_layout(w->cols, n_tok, act);
        launch_quantize(act, x, x_stride, w->cols, n_tok, scratch, st);
        launch_i8(w, act, scratch, n_tok, y, y_stride, scratch + l.bytes, st);
    }
    NNH_HIP(hipGetLastError());
    return NNH_OK;
}

// Work of the device argmax: the partial keys, then (Q4, fused path) the
// block sums of x.
bool argmax_fused(const nnh_weight* w, int act) { return act == NNH_ACT_F32 && w->dtype != NNH_BF16 && w->f32v2; }
size_t argmax_parts(const nnh_weight* w, int act) {
    return argmax_fused(w, act) ? (size_t)nnh::f32_v2_parts((int)w->rows) : nnh::argmax_partial_words(w->rows);
}

// Queue y = W x and the row of its first largest value into *out (device
// pointers; `work` holds argmax_parts words and, fused Q4, nb floats).
// Through the 8-lane kernel the first argmax stage is fused into the gemv.
int run_argmax(const nnh_weight* w, const float* x, float* y, uint8_t* work, uint64_t* out, int act,
               uint8_t* scratch, hipStream_t st) {
    uint64_t* part = (uint64_t*)work;
    if (argmax_fused(w, act)) {
        float* xsum = (float*)(work + align_up(argmax_parts(w, act) * 8));
        nnh::launch_gemv_f32_v2_argmax(w->dtype, w->fq, w->fs, w->bi, x, xsum, (int)w->rows, (int)w->nb,
                                       (int)w->nbp, y, part, st);
        nnh::launch_argmax_final(y, part, (int)argmax_parts(w, act), out, st, 0);
    } else {
        int rc = run_gemv(w, x, w->cols, y, w->rows, 1, act, scratch, st);
        if (rc) return rc;
        // BF16 with the 4-row kernel streams a running best from -inf
        // (kernels/mod.rs:384-406), the rest take the first-max argmax.
        nnh::launch_argmax(y, w->rows, part, out, st, w->dtype == NNH_BF16 && w->bpath == nnh::BF16_PATH_QUAD ? 1 : 0);
    }
    NNH_HIP(hipGetLastError());
    return NNH_OK;
}

size_t argmax_work_bytes(const nnh_weight* w, int act) {
    return align_up(argmax_parts(w, act) * 8) + (argmax_fused(w, act) && w->dtype == NNH_Q4S ? w->nb * 4 : 0);
}

size_t gemv_scratch_bytes(const nnh_weight* w, size_t n_tok, int act) {
    if (w->dtype == NNH_BF16) return 0;
    if (act == NNH_ACT_F32) return w->dtype == NNH_Q4S ? align_up(n_tok * w->nb * 4) : 0;
    return act_layout(w->cols, n_tok, act).bytes + i8_workspace_bytes(w, n_tok, act);
}

int check_call(const nnh_weight* w, size_t x_stride, size_t y_stride, size_t n_tok, int act) {
    int rc = check_weight(w);
    if (rc) return rc;
    if (act != NNH_ACT_F32 && act != NNH_ACT_I8 && act != NNH_ACT_MXI8)
        return fail(NNH_E_INVALID, "unknown activation mode");
    if (w->dtype == NNH_BF16 && act != NNH_ACT_F32)
        return fail(NNH_E_INVALID, "BF16 weights take f32 activations (the int8 path is for Q8_0 / Q4)");
    if (n_tok > 1 && y_stride < w->rows) return fail(NNH_E_INVALID, "gemv batch: y_stride < rows");
    if (n_tok > (size_t)1 << 20) return fail(NNH_E_INVALID, "gemv batch: too many vectors");
    if (act != NNH_ACT_F32 && n_tok * w->cols >= ((size_t)1 << 30))
        return fail(NNH_E_INVALID, "gemv batch: activations too large for the int8 path (n_tok * cols >= 2^30)");
    (void)x_stride;
    return NNH_OK;
}

int check_shape(int dtype, size_t rows, size_t cols) {
    if (dtype != NNH_Q8_0 && dtype != NNH_Q4S && dtype != NNH_BF16) return fail(NNH_E_INVALID, "unknown dtype");
    if (rows == 0 || cols == 0) return fail(NNH_E_INVALID, "empty matrix");
    if (dtype != NNH_BF16 && cols % 32 != 0) return fail(NNH_E_INVALID, "cols is not a multiple of 32");
    if (rows >= ((size_t)1 << 31) || cols >= ((size_t)1 << 31) || rows > ((size_t)1 << 62) / cols)
        return fail(NNH_E_INVALID, "matrix too large");
    return NNH_OK;
}

size_t raw_bytes_of(int dtype, size_t rows, size_t cols) {
    const size_t n = rows * cols;
    if (dtype == NNH_BF16) return 2 * n;
    return dtype == NNH_Q8_0 ? n + n / 16 : n / 2 + n / 8;
}

void release(nnh_weight* w) {
    if (w->raw) (void)hipFree(w->raw);
    if (w->fq) (void)hipFree(w->fq);
    if (w->fs) (void)hipFree(w->fs);
    if (w->sb) (void)hipFree(w->sb);
    if (w->swT) (void)hipFree(w->swT);
    if (w->bl) (void)hipFree(w->bl);
    if (w->wbi) (void)hipFree(w->wbi);
    delete w;
}

// Matrices from this many rows get the bit-exact path's 8-lane layout
// (measured faster from 14336 rows; matrices of at most 8192 rows keep the
// 16-lane layout that nnh_weight_f32_layout hands out).
#ifndef NNH_F32_V2_MIN_ROWS
#define NNH_F32_V2_MIN_ROWS 12288
#endif
constexpr size_t F32_V2_MIN_ROWS = NNH_F32_V2_MIN_ROWS;

// Derived layouts, built on the first call that reads them.
enum : unsigned {
    LAY_F32 = 1,  // fq + fs: the bit-exact f32 path
    LAY_SB = 2,   // Q4 sb: the int8 GEMV
    LAY_SWT = 4,  // swT: the MFMA kernels (few-token, GEMM)
    LAY_MX = 8,   // Q4 wbi: the MX GEMM's bias operand
};

// What a call with activation mode `act` over n_tok vectors reads.
unsigned layouts_for(const nnh_weight* w, int act, size_t n_tok) {
    if (w->dtype == NNH_BF16) return 0;
    if (act == NNH_ACT_F32) return LAY_F32;
    if (n_tok >= GEMM_MIN_TOKENS && act == NNH_ACT_MXI8) return LAY_SWT | LAY_MX;
    if (n_tok >= SKINNY_MIN_TOKENS) return LAY_SWT;
    return w->dtype == NNH_Q4S ? LAY_SB : 0;
}

// Allocate a weight's split layout (BF16: and its chain layout); caller
// holds g_mu.
int alloc_weight(int dtype, size_t rows, size_t cols, nnh_weight** out) {
    nnh_weight* w = new nnh_weight();
    w->dtype = dtype;
    w->device = g_device;
    w->rows = rows;
    w->cols = cols;
    const size_t rb = align_up(raw_bytes_of(dtype, rows, cols));
    hipError_t e = hipMalloc((void**)&w->raw, rb);
    w->dev_bytes = rb;
    if (e == hipSuccess && dtype == NNH_BF16) {
        w->bpath = nnh::bf16_path(rows, cols);
        const size_t lb = nnh::bf16_layout_bytes(w->bpath, rows, cols);
        if (lb) {
            e = hipMalloc((void**)&w->bl, align_up(lb));
            w->dev_bytes += align_up(lb);
        }
    }
    if (e != hipSuccess) {
        release(w);
        return fail(e == hipErrorOutOfMemory ? NNH_E_OOM : NNH_E_DEVICE,
                    std::string("weight alloc: ") + hipGetErrorString(e));
    }
    if (dtype != NNH_BF16) {
        const size_t n = rows * cols, nb = cols / 32;
        const size_t qbytes = dtype == NNH_Q8_0 ? n : n / 2;
        const size_t group = dtype == NNH_Q8_0 ? 8 : 16;
        w->nb = nb;
        w->nbp = (nb + group - 1) / group * group;
        w->f32v2 = rows >= F32_V2_MIN_ROWS && cols * 4 <= (size_t)nnh::F32_V2_MAX_LDS;
        w->qs = w->raw;
        w->sc = (const uint16_t*)(w->raw + qbytes);
        w->bi = dtype == NNH_Q4S ? (const uint16_t*)(w->raw + qbytes + (n / 32) * 2) : nullptr;
    }
    *out = w;
    return NNH_OK;
}

// Build the BF16 chain layout from `raw`, then wait for everything queued
// on the library stream for this weight (the upload copies or the encode
// kernel, every dtype); caller holds g_mu. On return the caller may free or
// reuse the source, and any stream may read `raw` (Q8_0 and Q4 derived
// layouts are built by prepare_locked when a call first needs them).
int finalize_weight(nnh_weight* w) {
    if (w->dtype == NNH_BF16)
        nnh::launch_relayout_bf16(w->bpath, (const uint16_t*)w->raw, w->bl, (int)w->rows, (int)w->cols, g_stream);
    hipError_t e;
    if ((e = hipGetLastError()) != hipSuccess || (e = hipStreamSynchronize(g_stream)) != hipSuccess)
        return fail(NNH_E_DEVICE, std::string("weight layouts: ") + hipGetErrorString(e));
    return NNH_OK;
}

// A derived layout's buffer; one left by an earlier call whose later
// allocation failed is reused, so a retry neither leaks nor double-counts.
int dev_alloc(nnh_weight* w, void** p, size_t bytes) {
    if (*p) return NNH_OK;
    const size_t b = align_up(bytes);
    hipError_t e = hipMalloc(p, b);
    if (e != hipSuccess)
        return fail(e == hipErrorOutOfMemory ? NNH_E_OOM : NNH_E_DEVICE,
                    std::string("weight layout alloc: ") + hipGetErrorString(e));
    w->dev_bytes += b;
    return NNH_OK;
}

// Build the derived layouts in `need` that `w` lacks, from its split layout
// (read-only since upload), on the library stream, and wait for them; caller
// holds g_mu. Nothing queued on any caller stream can read a layout before
// it exists, since the calls that read it are queued after this returns.
int prepare_locked(const nnh_weight* cw, unsigned need) {
    nnh_weight* w = const_cast<nnh_weight*>(cw);
    need &= ~w->ready;
    if (!need) return NNH_OK;
    int rc;
    const int rows = (int)w->rows, nb = (int)w->nb;
    if (need & LAY_F32) {
        if ((rc = dev_alloc(w, (void**)&w->fq, nnh::f32_quant_bytes(w->dtype, rows, nb, w->f32v2))) ||
            (rc = dev_alloc(w, (void**)&w->fs, w->rows * w->nbp * 2)))
            return rc;
        nnh::launch_relayout_f32(w->dtype, w->qs, w->sc, w->fq, w->fs, rows, nb, (int)w->nbp, w->f32v2, g_stream);
    }
    if ((need & LAY_SB) && w->dtype == NNH_Q4S) {
        if ((rc = dev_alloc(w, (void**)&w->sb, w->rows * w->nb * 4))) return rc;
        nnh::launch_pack_sb(w->sc, w->bi, w->sb, w->rows * w->nb, g_stream);
    }
    if (need & LAY_SWT) {
        // Q8 one spare block row (the MX GEMM loads scales in pairs of
        // blocks); for Q4 the bias table follows the scales.
        const size_t bytes = (size_t)nnh::gemm_rows_pad(rows) * 4 * (w->dtype == NNH_Q4S ? 2 * w->nb : w->nb + 1);
        if ((rc = dev_alloc(w, (void**)&w->swT, bytes))) return rc;
        nnh::launch_gemm_scales(w->sc, w->bi, w->swT, rows, nb, g_stream);
    }
    if ((need & LAY_MX) && w->dtype == NNH_Q4S) {
        if ((rc = dev_alloc(w, (void**)&w->wbi, nnh::mx_bias_bytes(rows, nb)))) return rc;
        nnh::launch_mx_bias(w->bi, rows, nb, w->wbi, g_stream);
    }
    hipError_t e;
    if ((e = hipGetLastError()) != hipSuccess || (e = hipStreamSynchronize(g_stream)) != hipSuccess)
        return fail(NNH_E_DEVICE, std::string("weight layouts: ") + hipGetErrorString(e));
    w->ready |= need;
    return NNH_OK;
}

int upload_parts(int dtype, const void* qs, const void* sc, const void* bi, size_t rows, size_t cols,
                 nnh_weight** out) {
    if (!out) return fail(NNH_E_INVALID, "nnh_upload: null out");
    *out = nullptr;
    int rc = check_shape(dtype, rows, cols);
    if (rc) return rc;
    if (!qs || (dtype != NNH_BF16 && !sc) || (dtype == NNH_Q4S && !bi)) return fail(NNH_E_INVALID, "nnh_upload: null data");
    std::lock_guard<std::mutex> g(g_mu);
    if ((rc = ensure_locked())) return rc;
    nnh_weight* w;
    if ((rc = alloc_weight(dtype, rows, cols, &w))) return rc;
    const size_t n = rows * cols;
    const size_t qbytes = dtype == NNH_BF16 ? 2 * n : dtype == NNH_Q8_0 ? n : n / 2, tbytes = (n / 32) * 2;
    hipError_t e;
    if ((e = hipMemcpyAsync(w->raw, qs, qbytes, hipMemcpyHostToDevice, g_stream)) != hipSuccess ||
        (dtype != NNH_BF16 &&
         (e = hipMemcpyAsync(w->raw + qbytes, sc, tbytes, hipMemcpyHostToDevice, g_stream)) != hipSuccess) ||
        (dtype == NNH_Q4S &&
         (e = hipMemcpyAsync(w->raw + qbytes + tbytes, bi, tbytes, hipMemcpyHostToDevice, g_stream)) != hipSuccess)) {
        release(w);
        return fail(NNH_E_DEVICE, std::string("nnh_upload: copy: ") + hipGetErrorString(e));
    }
    if ((rc = finalize_weight(w))) {
        release(w);
        return rc;
    }
    *out = w;
    return NNH_OK;
}

}  // namespace

extern "C" {

int nnh_init(int device) {
    std::lock_guard<std::mutex> g(g_mu);
    return init_locked(device);
}

const char* nnh_last_error(void) { return t_err.c_str(); }

int nnh_upload_q8_0(const int8_t* qs, const uint16_t* scales, size_t rows, size_t cols, nnh_weight** out) {
    return upload_parts(NNH_Q8_0, qs, scales, nullptr, rows, cols, out);
}

int nnh_upload_q4(const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, size_t rows, size_t cols,
                  nnh_weight** out) {
    return upload_parts(NNH_Q4S, qs, scales, biases, rows, cols, out);
}

int nnh_upload_bf16(const uint16_t* w, size_t rows, size_t cols, nnh_weight** out) {
    return upload_parts(NNH_BF16, w, nullptr, nullptr, rows, cols, out);
}

int nnh_upload(int dtype, const void* data, size_t rows, size_t cols, nnh_weight** out) {
    if (!data) return fail(NNH_E_INVALID, "nnh_upload: null data");
    const uint8_t* p = (const uint8_t*)data;
    size_t n = rows * cols;
    if (dtype == NNH_BF16) return upload_parts(dtype, p, nullptr, nullptr, rows, cols, out);
    if (dtype == NNH_Q8_0) return upload_parts(dtype, p, p + n, nullptr, rows, cols, out);
    if (dtype == NNH_Q4S) return upload_parts(dtype, p, p + n / 2, p + n / 2 + n / 16, rows, cols, out);
    return fail(NNH_E_INVALID, "nnh_upload: unknown dtype");
}

void nnh_free(nnh_weight* w) {
    if (!w) return;
    std::lock_guard<std::mutex> g(g_mu);
    (void)hipSetDevice(w->device);
    (void)hipDeviceSynchronize();
    release(w);
}

int nnh_encode_dev(int dtype, const float* w, size_t rows, size_t cols, nnh_weight** out, void* stream) {
    if (!out) return fail(NNH_E_INVALID, "nnh_encode_dev: null out");
    *out = nullptr;
    int rc = check_shape(dtype, rows, cols);
    if (rc) return rc;
    if (!w) return fail(NNH_E_INVALID, "nnh_encode_dev: null weights");
    std::lock_guard<std::mutex> g(g_mu);
    if ((rc = ensure_locked())) return rc;
    NNH_HIP(hipStreamSynchronize((hipStream_t)stream));  // w may come from work queued on `stream`
    nnh_weight* d;
    if ((rc = alloc_weight(dtype, rows, cols, &d))) return rc;
    if (dtype == NNH_BF16)
        nnh::launch_encode_bf16(w, rows * cols, (uint16_t*)d->raw, g_stream);
    else
        nnh::launch_encode(dtype, w, rows * cols, d->raw, (uint16_t*)d->sc, (uint16_t*)d->bi, g_stream);
    if ((rc = finalize_weight(d))) {
        release(d);
        return rc;
    }
    *out = d;
    return NNH_OK;
}

// dequantize_to_f32's conditions (kernels/quant.rs:112-124).
int check_blocks(uint32_t type, size_t nbytes, size_t n) {
    size_t bytes, per;
    if (!nnh::ggml_block(type, &bytes, &per)) return fail(NNH_E_INVALID, "dequantize: type not decodable");
    if (n % per != 0) return fail(NNH_E_INVALID, "dequantize: not a whole number of blocks");
    if (nbytes / bytes < n / per) return fail(NNH_E_INVALID, "dequantize: fewer blocks than values");
    return NNH_OK;
}

int nnh_dequantize_dev(uint32_t ggml_type, const void* blocks, size_t nbytes, float* dst, size_t n, void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if ((rc = check_blocks(ggml_type, nbytes, n))) return rc;
    if (n == 0) return NNH_OK;
    if (!blocks || !dst) return fail(NNH_E_INVALID, "dequantize: null pointer");
    nnh::launch_dequantize(ggml_type, (const uint8_t*)blocks, n, dst, (hipStream_t)stream);
    NNH_HIP(hipGetLastError());
    return NNH_OK;
}

int nnh_upload_gguf(uint32_t ggml_type, const void* blocks, size_t nbytes, size_t rows, size_t cols, int dtype,
                    nnh_weight** out) {
    if (!out) return fail(NNH_E_INVALID, "nnh_upload_gguf: null out");
    *out = nullptr;
    int rc = check_shape(dtype, rows, cols);
    if (rc) return rc;
    if ((rc = check_blocks(ggml_type, nbytes, rows * cols))) return rc;
    if (!blocks) return fail(NNH_E_INVALID, "nnh_upload_gguf: null blocks");
    size_t bytes, per;
    nnh::ggml_block(ggml_type, &bytes, &per);
    const size_t n = rows * cols, used = n / per * bytes;
    uint8_t* dblk = nullptr;
    float* df = nullptr;
    {
        std::lock_guard<std::mutex> g(g_mu);
        if ((rc = ensure_locked())) return rc;
        hipError_t e;
        if ((e = hipMalloc((void**)&dblk, align_up(used))) != hipSuccess ||
            (e = hipMalloc((void**)&df, align_up(n * 4))) != hipSuccess) {
            if (dblk) (void)hipFree(dblk);
            return fail(e == hipErrorOutOfMemory ? NNH_E_OOM : NNH_E_DEVICE,
                        std::string("nnh_upload_gguf: alloc: ") + hipGetErrorString(e));
        }
        if ((e = hipMemcpyAsync(dblk, blocks, used, hipMemcpyHostToDevice, g_stream)) != hipSuccess) {
            (void)hipFree(dblk);
            (void)hipFree(df);
            return fail(NNH_E_DEVICE, std::string("nnh_upload_gguf: copy: ") + hipGetErrorString(e));
        }
        nnh::launch_dequantize(ggml_type, dblk, n, df, g_stream);
        if ((e = hipGetLastError()) != hipSuccess || (e = hipStreamSynchronize(g_stream)) != hipSuccess) {
            (void)hipFree(dblk);
            (void)hipFree(df);
            return fail(NNH_E_DEVICE, std::string("nnh_upload_gguf: decode: ") + hipGetErrorString(e));
        }
        (void)hipFree(dblk);
    }
    // Re-encode (load.rs:182-206) as nnh_encode_dev does; g_stream is idle.
    rc = nnh_encode_dev(dtype, df, rows, cols, out, nullptr);
    std::lock_guard<std::mutex> g(g_mu);
    (void)hipFree(df);
    return rc;
}

int nnh_weight_download(const nnh_weight* w, void* data, size_t bytes) {
    if (!w || !data) return fail(NNH_E_INVALID, "nnh_weight_download: null pointer");
    const size_t need = raw_bytes_of(w->dtype, w->rows, w->cols);
    if (bytes < need) return fail(NNH_E_INVALID, "nnh_weight_download: buffer too small");
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    NNH_HIP(hipMemcpyAsync(data, w->raw, need, hipMemcpyDeviceToHost, g_stream));
    NNH_HIP(hipStreamSynchronize(g_stream));
    return NNH_OK;
}

const void* nnh_weight_device_data(const nnh_weight* w) { return w ? (const void*)w->raw : nullptr; }

size_t nnh_argmax_work_bytes(size_t n) { return nnh::argmax_partial_words(n) * 8; }

int nnh_argmax_dev(const float* v, size_t n, void* work, uint64_t* out_row, void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if (n == 0 || n >= ((size_t)1 << 32)) return fail(NNH_E_INVALID, "argmax: n must be in [1, 2^32)");
    if (!v || !work || !out_row) return fail(NNH_E_INVALID, "argmax: null pointer");
    nnh::launch_argmax(v, n, (uint64_t*)work, out_row, (hipStream_t)stream);
    NNH_HIP(hipGetLastError());
    return NNH_OK;
}

int nnh_weight_f32_layout(const nnh_weight* w, nnh_f32_layout* out) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if ((rc = check_weight(w))) return rc;
    if (!out) return fail(NNH_E_INVALID, "f32 layout: null output");
    if (w->dtype == NNH_BF16) return fail(NNH_E_INVALID, "f32 layout: BF16 weight (no quant layout)");
    if (w->f32v2) return fail(NNH_E_INVALID, "f32 layout: tall weight (8-lane layout)");
    if ((rc = prepare_locked(w, LAY_F32))) return rc;
    *out = nnh_f32_layout{w->fq, w->fs, w->bi, w->rows, w->cols, w->nb, w->nbp, w->dtype};
    return NNH_OK;
}

int nnh_weight_prepare(const nnh_weight* w, int act, size_t n_tok) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if ((rc = check_call(w, 0, w ? w->rows : 0, n_tok, act))) return rc;
    return prepare_locked(w, layouts_for(w, act, n_tok));
}

size_t nnh_weight_device_bytes(const nnh_weight* w) {
    if (!w) return 0;
    std::lock_guard<std::mutex> g(g_mu);
    return w->dev_bytes;
}

int nnh_weight_info(const nnh_weight* w, int* dtype, size_t* rows, size_t* cols) {
    if (!w) return fail(NNH_E_INVALID, "null weight");
    if (dtype) *dtype = w->dtype;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    return NNH_OK;
}

int nnh_gemv_batch(const nnh_weight* w, const float* x, size_t x_stride, float* y, size_t y_stride, size_t n_tok,
                   int act) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if ((rc = check_call(w, x_stride, y_stride, n_tok, act))) return rc;
    if (n_tok == 0) return NNH_OK;
    if (!x || !y) return fail(NNH_E_INVALID, "gemv: null x or y");
    const size_t xs = n_tok > 1 ? x_stride : w->cols;
    const size_t ys = n_tok > 1 ? y_stride : w->rows;
    const size_t x_elems = (n_tok - 1) * xs + w->cols;
    const size_t y_elems = (n_tok - 1) * ys + w->rows;
    const size_t off_y = align_up(x_elems * 4);
    const size_t off_s = off_y + align_up(y_elems * 4);
    uint8_t *s, *h;
    if ((rc = prepare_locked(w, layouts_for(w, act, n_tok)))) return rc;
    if ((rc = scratch_locked(g_stream, off_s + gemv_scratch_bytes(w, n_tok, act), &s))) return rc;
    if ((rc = pinned_locked(off_s, &h))) return rc;
    float* dx = (float*)s;
    float* dy = (float*)(s + off_y);
    // Through pinned staging: the DMA engines copy pinned memory directly,
    // where pageable copies go through the runtime's own bounce buffers.
    std::memcpy(h, x, x_elems * 4);
    NNH_HIP(hipMemcpyAsync(dx, h, x_elems * 4, hipMemcpyHostToDevice, g_stream));
    if ((rc = run_gemv(w, dx, xs, dy, ys, n_tok, act, s + off_s, g_stream))) return rc;
    float* hy = (float*)(h + off_y);
    NNH_HIP(hipMemcpyAsync(hy, dy, y_elems * 4, hipMemcpyDeviceToHost, g_stream));
    NNH_HIP(hipStreamSynchronize(g_stream));
    // Only each vector's rows: the reference leaves the stride gaps alone.
    for (size_t t = 0; t < n_tok; ++t) std::memcpy(y + t * ys, hy + t * ys, w->rows * 4);
    return NNH_OK;
}

int nnh_model_gemv(const nnh_weight* w, const float* x, float* y, int act) {
    return nnh_gemv_batch(w, x, w ? w->cols : 0, y, w ? w->rows : 0, 1, act);
}

int nnh_model_argmax(const nnh_weight* w, const float* x, size_t* out_row, int act) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if ((rc = check_call(w, 0, 0, 1, act))) return rc;
    if (!x || !out_row) return fail(NNH_E_INVALID, "argmax: null x or out");
    if (w->rows >= ((size_t)1 << 32)) return fail(NNH_E_INVALID, "argmax: too many rows");
    const size_t off_y = align_up(w->cols * 4);
    const size_t off_p = off_y + align_up(w->rows * 4);
    const size_t off_o = off_p + align_up(argmax_work_bytes(w, act));
    const size_t off_s = off_o + ALIGN;
    uint8_t *s, *h;
    if ((rc = prepare_locked(w, layouts_for(w, act, 1)))) return rc;
    if ((rc = scratch_locked(g_stream, off_s + gemv_scratch_bytes(w, 1, act), &s))) return rc;
    if ((rc = pinned_locked(off_y + ALIGN, &h))) return rc;
    float* dx = (float*)s;
    float* dy = (float*)(s + off_y);
    uint64_t* dout = (uint64_t*)(s + off_o);
    std::memcpy(h, x, w->cols * 4);
    NNH_HIP(hipMemcpyAsync(dx, h, w->cols * 4, hipMemcpyHostToDevice, g_stream));
    if ((rc = run_argmax(w, dx, dy, s + off_p, dout, act, s + off_s, g_stream))) return rc;
    uint64_t* hidx = (uint64_t*)(h + off_y);
    NNH_HIP(hipMemcpyAsync(hidx, dout, 8, hipMemcpyDeviceToHost, g_stream));
    NNH_HIP(hipStreamSynchronize(g_stream));
    *out_row = (size_t)*hidx;
    return NNH_OK;
}

size_t nnh_model_argmax_work_bytes(const nnh_weight* w) { return w ? argmax_work_bytes(w, NNH_ACT_F32) : 0; }

int nnh_model_argmax_dev(const nnh_weight* w, const float* x, float* logits, void* work, uint64_t* out_row,
                         void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if ((rc = check_call(w, 0, 0, 1, NNH_ACT_F32))) return rc;
    if (w->rows >= ((size_t)1 << 32)) return fail(NNH_E_INVALID, "argmax: too many rows");
    if (!x || !logits || !work || !out_row) return fail(NNH_E_INVALID, "argmax: null pointer");
    uint8_t* s = nullptr;
    if ((rc = prepare_locked(w, layouts_for(w, NNH_ACT_F32, 1)))) return rc;
    const size_t need = argmax_fused(w, NNH_ACT_F32) ? 0 : gemv_scratch_bytes(w, 1, NNH_ACT_F32);
    if (need && (rc = scratch_locked((hipStream_t)stream, need, &s))) return rc;
    return run_argmax(w, x, logits, (uint8_t*)work, out_row, NNH_ACT_F32, s, (hipStream_t)stream);
}

int nnh_gemv_batch_dev(const nnh_weight* w, const float* x, size_t x_stride, float* y, size_t y_stride,
                       size_t n_tok, int act, void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if ((rc = check_call(w, x_stride, y_stride, n_tok, act))) return rc;
    if (n_tok == 0) return NNH_OK;
    if (!x || !y) return fail(NNH_E_INVALID, "gemv: null x or y");
    uint8_t* s = nullptr;
    if ((rc = prepare_locked(w, layouts_for(w, act, n_tok)))) return rc;
    size_t need = gemv_scratch_bytes(w, n_tok, act);
    if (need && (rc = scratch_locked((hipStream_t)stream, need, &s))) return rc;
    const size_t xs = n_tok > 1 ? x_stride : w->cols;
    const size_t ys = n_tok > 1 ? y_stride : w->rows;
    return run_gemv(w, x, xs, y, ys, n_tok, act, s, (hipStream_t)stream);
}

int nnh_gemv_rmsnorm_act_dev(const nnh_weight* w, int act, const float* x, const float* r, const float* gamma,
                             float eps, float* x_out, float* rec, float* normed, float* y, void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if (act != NNH_ACT_F32 && act != NNH_ACT_I8)
        return fail(NNH_E_INVALID, "gemv rmsnorm: activation mode is not NNH_ACT_F32 or NNH_ACT_I8");
    if ((rc = check_call(w, w ? w->cols : 0, w ? w->rows : 0, 1, act))) return rc;
    if (!x || !gamma || !normed || !y) return fail(NNH_E_INVALID, "gemv rmsnorm: null x, gamma, normed or y");
    if (w->cols > 16384) return fail(NNH_E_INVALID, "gemv rmsnorm: more than 16384 columns");
    const auto overlaps = [&](const float* a, const float* b) { return a && b && a < b + w->cols && b < a + w->cols; };
    if (overlaps(x_out, x) || overlaps(x_out, r) || overlaps(rec, x) || overlaps(rec, r))
        return fail(NNH_E_INVALID, "gemv rmsnorm: x_out / rec overlap x or r");
    if ((rc = prepare_locked(w, layouts_for(w, act, 1)))) return rc;
    const hipStream_t st = (hipStream_t)stream;
    const nnh::NormIn nrm{x, r, gamma, x_out, rec, eps};
    if (w->dtype != NNH_BF16) {
        const bool fused =
            act == NNH_ACT_F32
                ? nnh::launch_gemv_f32_norm(w->dtype, w->fq, w->fs, w->bi, nrm, (int)w->rows, (int)w->nb,
                                            (int)w->nbp, y, w->f32v2, st)
                : nnh::launch_gemv_i8_norm(w->dtype, w->qs, w->sc, w->sb, nrm, (int)w->rows, (int)w->nb, y, st);
        if (fused) {
            NNH_HIP(hipGetLastError());
            return NNH_OK;
        }
    }
    uint8_t* s = nullptr;
    const size_t need = gemv_scratch_bytes(w, 1, act);
    if (need && (rc = scratch_locked(st, need, &s))) return rc;
    nnh::launch_rmsnorm_vec(nrm, (int)w->cols, normed, st);
    NNH_HIP(hipGetLastError());
    return run_gemv(w, normed, w->cols, y, w->rows, 1, act, s, st);
}

int nnh_gemv_rmsnorm_dev(const nnh_weight* w, const float* x, const float* r, const float* gamma, float eps,
                         float* x_out, float* rec, float* normed, float* y, void* stream) {
    return nnh_gemv_rmsnorm_act_dev(w, NNH_ACT_F32, x, r, gamma, eps, x_out, rec, normed, y, stream);
}


int nnh_gemv_batch_dev_noalloc(const nnh_weight* w, const float* x, size_t x_stride, float* y, size_t y_stride,
                               size_t n_tok, int act, void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    if (g_device < 0 || !g_noalloc) return fail(NNH_E_STATE, "gemv noalloc: call nnh_init first");
    NNH_HIP(hipSetDevice(g_device));
    int rc = check_call(w, x_stride, y_stride, n_tok, act);
    if (rc) return rc;
    if (n_tok == 0) return NNH_OK;
    if (!x || !y) return fail(NNH_E_INVALID, "gemv noalloc: null x or y");
    const unsigned need = layouts_for(w, act, n_tok);
    if ((w->ready & need) != need)
        return fail(NNH_E_STATE, "gemv noalloc: the weight's layouts for this mode and batch are not built "
                                 "(nnh_weight_prepare, or one call of nnh_gemv_batch_dev, builds them)");
    const size_t bytes = gemv_scratch_bytes(w, n_tok, act);
    if (bytes > (size_t)NNH_NOALLOC_SCRATCH_BYTES)
        return fail(NNH_E_INVALID, "gemv noalloc: this call needs " + std::to_string(bytes) +
                                       " bytes of scratch, more than the no-alloc maximum of " +
                                       std::to_string((size_t)NNH_NOALLOC_SCRATCH_BYTES));
    const size_t xs = n_tok > 1 ? x_stride : w->cols;
    const size_t ys = n_tok > 1 ? y_stride : w->rows;
    return run_gemv(w, x, xs, y, ys, n_tok, act, g_noalloc, (hipStream_t)stream);
}

int nnh_act_layout_ex(int act, size_t cols, size_t n_tok, size_t* off_s, size_t* off_sx, size_t* bytes) {
    if (act != NNH_ACT_I8 && act != NNH_ACT_MXI8) return fail(NNH_E_INVALID, "act layout: not an int8 mode");
    if (cols % 32 != 0) return fail(NNH_E_INVALID, "act layout: cols is not a multiple of 32");
    ActLayout l = act_layout(cols, n_tok, act);
    if (off_s) *off_s = l.off_s;
    if (off_sx) *off_sx = l.off_sx;
    if (bytes) *bytes = l.bytes;
    return NNH_OK;
}

int nnh_act_layout(size_t cols, size_t n_tok, size_t* off_s, size_t* off_sx, size_t* bytes) {
    return nnh_act_layout_ex(NNH_ACT_I8, cols, n_tok, off_s, off_sx, bytes);
}

int nnh_quantize_act_ex_dev(int act, const float* x, size_t x_stride, size_t cols, size_t n_tok, void* buf,
                            void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if (act != NNH_ACT_I8 && act != NNH_ACT_MXI8) return fail(NNH_E_INVALID, "quantize: not an int8 mode");
    if (cols == 0 || cols % 32 != 0) return fail(NNH_E_INVALID, "quantize: cols is not a positive multiple of 32");
    if (n_tok == 0) return NNH_OK;
    if (!x || !buf) return fail(NNH_E_INVALID, "quantize: null pointer");
    if (cols >= ((size_t)1 << 31) || n_tok * cols >= ((size_t)1 << 30)) return fail(NNH_E_INVALID, "quantize: too large");
    launch_quantize(act, x, n_tok > 1 ? x_stride : cols, cols, n_tok, (uint8_t*)buf, (hipStream_t)stream);
    NNH_HIP(hipGetLastError());
    return NNH_OK;
}

int nnh_quantize_act_dev(const float* x, size_t x_stride, size_t cols, size_t n_tok, void* act, void* stream) {
    return nnh_quantize_act_ex_dev(NNH_ACT_I8, x, x_stride, cols, n_tok, act, stream);
}

int nnh_gemv_act_dev(const nnh_weight* w, int act, const void* buf, size_t n_tok, float* y, size_t y_stride,
                     void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if (act != NNH_ACT_I8 && act != NNH_ACT_MXI8) return fail(NNH_E_INVALID, "gemv_act: not an int8 mode");
    if ((rc = check_call(w, 0, y_stride, n_tok, act))) return rc;
    if (n_tok == 0) return NNH_OK;
    if (!buf || !y) return fail(NNH_E_INVALID, "gemv_act: null pointer");
    uint8_t* ws = nullptr;
    if ((rc = prepare_locked(w, layouts_for(w, act, n_tok)))) return rc;
    const size_t wsb = i8_workspace_bytes(w, n_tok, act);
    if (wsb && (rc = scratch_locked((hipStream_t)stream, wsb, &ws))) return rc;
    launch_i8(w, act, (const uint8_t*)buf, n_tok, y, n_tok > 1 ? y_stride : w->rows, ws, (hipStream_t)stream);
    NNH_HIP(hipGetLastError());
    return NNH_OK;
}

int nnh_gemv_i8_dev(const nnh_weight* w, const void* act, size_t n_tok, float* y, size_t y_stride, void* stream) {
    return nnh_gemv_act_dev(w, NNH_ACT_I8, act, n_tok, y, y_stride, stream);
}

int nnh_block_dots_dev(const nnh_weight* w, const void* act, size_t n_tok, int32_t* P, void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if ((rc = check_weight(w))) return rc;
    if (w->dtype == NNH_BF16) return fail(NNH_E_INVALID, "block_dots: BF16 weight (no int8 blocks)");
    if (n_tok == 0) return NNH_OK;
    if (!act || !P) return fail(NNH_E_INVALID, "block_dots: null pointer");
    nnh::launch_block_dots(w->dtype, w->qs, (const int8_t*)act, (int)w->rows, (int)w->nb, (int)n_tok, P,
                           (hipStream_t)stream);
    NNH_HIP(hipGetLastError());
    return NNH_OK;
}

int nnh_stream_reserve(const nnh_weight* w, int act, size_t n_tok, void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    if ((rc = check_call(w, 0, w ? w->rows : 0, n_tok, act))) return rc;
    if ((rc = prepare_locked(w, layouts_for(w, act, n_tok)))) return rc;
    const size_t need = n_tok ? gemv_scratch_bytes(w, n_tok, act) : 0;
    uint8_t* s = nullptr;
    if (need && (rc = scratch_locked((hipStream_t)stream, need, &s))) return rc;
    return NNH_OK;
}

int nnh_stream_release(void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    auto it = g_scratch.find((hipStream_t)stream);
    if (it == g_scratch.end()) return NNH_OK;
    NNH_HIP(hipStreamSynchronize((hipStream_t)stream));
    for (uint8_t* p : it->second.retired) (void)hipFree(p);
    if (it->second.p) (void)hipFree(it->second.p);
    g_scratch.erase(it);
    return NNH_OK;
}

int nnh_sync(void* stream) {
    std::lock_guard<std::mutex> g(g_mu);
    int rc = ensure_locked();
    if (rc) return rc;
    NNH_HIP(hipStreamSynchronize((hipStream_t)stream));
    return NNH_OK;
}

}  // extern "C"
