/*
 * nncpu_hip.h — the C-ABI of libnncpu_hip.so, the MI355X (gfx950) quantized
 * matmul that sits behind nncpu's matmul dispatch.
 *
 * The reference (ZacWalk/nncpu, Rust) dispatches every weight matmul through
 * two functions that read a `Tensor`'s dtype and call its CPU kernels:
 *
 *   model_gemv  crates/nncpu/src/model/mod.rs:417-444      (one vector)
 *   gemv_batch  crates/nncpu/src/model/forward.rs:15-58    (n_tok vectors, one weight pass)
 *
 * and greedy decoding reads the lm_head through model_argmax
 * (model/forward.rs:989-1011). This header replaces those three for the
 * Q8_0 and Q4 ("Q4S") split layouts (crates/nncpu/src/runtime.rs:52-63,
 * 136-164) and for BF16 weights (DType::BF16, Tensor::bf16()). Weights are uploaded once after load (model/load.rs:1266-1287)
 * and freed when the model drops (model/mod.rs:342-348).
 *
 * Plain C types only. Every function returns NNH_OK or an NNH_E_* code;
 * nnh_last_error() gives the calling thread's last message. All entry points
 * are thread-safe. Host-buffer calls are synchronous: y is ready on return,
 * as the reference's kernels are.
 */
#ifndef NNCPU_HIP_H
#define NNCPU_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. The Rust wrapper maps NNH_E_INVALID to a panic, as the
 * reference panics on violated kernel preconditions (kernels/mod.rs:12-14,
 * 412-415); NNH_E_OOM to ErrorKind::OutOfMemory (error.rs:8-23); and
 * NNH_E_DEVICE to an Io-like error. */
enum {
    NNH_OK = 0,
    NNH_E_INVALID = 1,
    NNH_E_OOM = 2,
    NNH_E_DEVICE = 3,
    NNH_E_STATE = 4
};

/* Weight formats: nncpu's DType::Q8_0, DType::Q4S and DType::BF16
 * (runtime.rs:52-63). BF16 weights take f32 activations only; the loader
 * keeps any matrix whose rows are not whole 32-element blocks in BF16
 * (model/load.rs:302-303), so a BF16 matrix may have any width. */
enum {
    NNH_Q8_0 = 1,
    NNH_Q4S = 2,
    NNH_BF16 = 3
};

/* Activation modes of a matmul call.
 *   NNH_ACT_F32: f32 activations, as the reference. Every output is
 *     bit-identical to nncpu's CPU kernels (kernels/scalar.rs:626-742,
 *     kernels/avx2.rs:1256-1521), and a batched call gives each vector the
 *     bits of a single-vector call.
 *   NNH_ACT_I8: each activation vector is quantized on the device with
 *     nncpu's own Q8_0 encoder (kernels/quant.rs:31-60) to int8 blocks of 32
 *     with a BF16 scale; the kernels form the exact int32 block dot products
 *     and scale them in f64. The result is the f32 rounding of the exact
 *     product of the dequantized weights and activations (from 17 vectors:
 *     within the f32 roundings of 8-block chunks of it, see the GEMM).
 *   NNH_ACT_MXI8: int8 blocks of 32 with a power-of-two scale (the OCP
 *     MXINT8 block; the scale still stored as BF16 bits): the least 2^E
 *     with 127 * 2^E >= max |x| of the block, q = rint(x / 2^E). Same exact
 *     block dots and f64 scaling as NNH_ACT_I8 (same buffer layout, plus
 *     BF16 operands), with which 17 or more vectors run on the BF16 matrix
 *     unit exactly: q_x 2^E and every weight quant are BF16 values, so each
 *     block dot comes out of the MFMA exact and the scaling costs one FMA
 *     per output and block. No counterpart in the reference, which never
 *     quantizes activations; an extension of the int8 path for prefill. */
enum {
    NNH_ACT_F32 = 0,
    NNH_ACT_I8 = 1,
    NNH_ACT_MXI8 = 2
};

typedef struct nnh_weight nnh_weight;

/* Select and initialise `device` for this process. Idempotent; a second call
 * with another device fails with NNH_E_STATE. */
int nnh_init(int device);

/* The calling thread's last error message ("" when none). */
const char* nnh_last_error(void);

/* Upload a matrix of `rows` x `cols` (cols % 32 == 0), one row per output,
 * from the split layout the reference's Tensor::q8()/q4() views
 * (runtime.rs:136-164). The host copy is not retained.
 *   nnh_upload_q8_0: qs[rows*cols], scales[rows*cols/32] (BF16 bits).
 *   nnh_upload_q4:   qs[rows*cols/2] (byte i of a block: element i low
 *                    nibble, element i+16 high), scales and biases
 *                    [rows*cols/32] (BF16 bits).
 *   nnh_upload:      one buffer as Tensor.data points at it (BF16: the
 *                    rows*cols values).
 * nnh_upload_bf16 (no 32-column condition): w[rows*cols] BF16 bits, row-major,
 * as Tensor::bf16() views them. Its matmuls are bit-identical to nncpu's
 * gemv_bf16 / gemv_bf16_batch (kernels/mod.rs:337-360, 454-485): the 4-row
 * kernel when rows % 4 == 0 (scalar.rs:555-571), the 1-row kernel otherwise
 * (scalar.rs:573-591), the f64 fallback when cols % 8 != 0 (mod.rs:556-564). */
int nnh_upload_q8_0(const int8_t* qs, const uint16_t* scales, size_t rows, size_t cols, nnh_weight** out);
int nnh_upload_q4(const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, size_t rows, size_t cols,
                  nnh_weight** out);
int nnh_upload(int dtype, const void* data, size_t rows, size_t cols, nnh_weight** out);
int nnh_upload_bf16(const uint16_t* w, size_t rows, size_t cols, nnh_weight** out);

/* Encode f32 weights (device memory, rows x cols row-major) with nncpu's
 * load-time re-encoder (kernels/quant.rs:31-95, as model/load.rs:182-206
 * calls it; BF16: f32_to_bf16 per value, load.rs:198-202), bit for bit,
 * straight into a device weight. Waits for `stream` first; synchronous. */
int nnh_encode_dev(int dtype, const float* w, size_t rows, size_t cols, nnh_weight** out, void* stream);

/* Load-time GGUF decoding on the device (kernels/quant.rs:97-156,
 * dequantize_to_f32), bit for bit: ggml types F32 (0), F16 (1), BF16 (30),
 * Q4_0 (2), Q4_1 (3), Q5_0 (6), Q5_1 (7), Q8_0 (8), Q4_K (12), Q5_K (13),
 * Q6_K (14). NNH_E_INVALID, dst untouched, for other types, when n is not a
 * whole number of blocks or `nbytes` holds fewer blocks than n needs.
 *   nnh_dequantize_dev: device blocks -> device dst[0..n), asynchronous on
 *                       `stream`.
 *   nnh_upload_gguf:    host blocks of one rows x cols matrix -> decoded on
 *                       the device -> re-encoded to `dtype` (NNH_Q8_0,
 *                       NNH_Q4S, NNH_BF16) as model/load.rs:182-206 does on
 *                       the CPU -> a new weight. Synchronous. */
int nnh_dequantize_dev(uint32_t ggml_type, const void* blocks, size_t nbytes, float* dst, size_t n, void* stream);
int nnh_upload_gguf(uint32_t ggml_type, const void* blocks, size_t nbytes, size_t rows, size_t cols, int dtype,
                    nnh_weight** out);

/* Copy a weight back to the host in nncpu's split layout (`bytes` >= the
 * layout's size: Q8_0 n + n/16, Q4 n/2 + n/8, BF16 2n for n = rows*cols). */
int nnh_weight_download(const nnh_weight* w, void* data, size_t bytes);

/* Release a weight (NULL is a no-op). */
void nnh_free(nnh_weight* w);

/* Shape and format of an uploaded weight. */
int nnh_weight_info(const nnh_weight* w, int* dtype, size_t* rows, size_t* cols);

/* Device memory of a weight. An upload holds nncpu's split layout only
 * (Q8_0 1.0625 B per weight, Q4 0.625; BF16 2 B plus its chain layout);
 * each activation mode builds the layouts its kernels read on the first call
 * that needs them, once (the upload's owner pays for the modes it uses):
 *   NNH_ACT_F32            Q8_0 +1.0625 B, Q4 +0.5625 B (per-lane quant groups,
 *                          padded scales)
 *   int8, 1..3 vectors     Q4 +0.125 B (packed scale | bias), Q8_0 nothing
 *   int8, 4 and more       +0.125 B Q8_0, +0.25 B Q4 (block-major f32 scales,
 *                          Q4 biases)
 *   NNH_ACT_MXI8, 17 and more vectors: as int8 with 4 and more, Q4 +0.125 B
 *                          more (BF16 biases); the quants are read in place
 * nnh_weight_prepare builds those of a call (act, n_tok) ahead of time, for
 * callers that capture calls into HIP graphs (a first call inside a capture
 * would allocate and synchronise the library's own stream there) or that
 * must not allocate later. nnh_weight_device_bytes gives the bytes held now.
 * No counterpart in the reference, whose kernels read the split layout. */
int nnh_weight_prepare(const nnh_weight* w, int act, size_t n_tok);
size_t nnh_weight_device_bytes(const nnh_weight* w);

/* Device address of the weight's split layout as uploaded (runtime.rs:136-164:
 * quants, then BF16 scales, then Q4 biases), read-only, valid until
 * nnh_free: the device form of Tensor::data, for callers that read rows
 * directly, as the embedding lookup does with the tied token_embd
 * (model/mod.rs:448-460). NULL for a NULL weight. */
const void* nnh_weight_device_data(const nnh_weight* w);

/* The bit-exact f32 path's device layout of a weight: the quants regrouped
 * per lane (16 lanes per row: Q8_0 groups of 8 blocks, lane j's 16 bytes
 * holding elements j and j + 16 of each block; Q4 groups of 16 blocks, lane
 * j's 16 bytes holding byte j of each), the BF16 scale rows padded to `nbp`
 * blocks, and the Q4 biases as uploaded. For callers that fuse their own
 * work around that matmul, as the device-resident decode step does; no
 * counterpart in the reference, whose forward calls the matmul per weight.
 * NNH_E_INVALID when the weight is tall (12288 rows or more with x of at
 * most 64 KB: those take the 8-lane layout instead). Read-only, valid until
 * nnh_free. */
typedef struct {
    const void* quants;
    const uint16_t* scales;
    const uint16_t* biases; /* Q4 only, else NULL */
    size_t rows, cols, nb, nbp;
    int dtype;
} nnh_f32_layout;
int nnh_weight_f32_layout(const nnh_weight* w, nnh_f32_layout* out);

/* model_gemv (model/mod.rs:417-444): y[0..rows) = W x[0..cols).
 * Host buffers; synchronous. */
int nnh_model_gemv(const nnh_weight* w, const float* x, float* y, int act);

/* gemv_batch (model/forward.rs:15-58) and kernels::gemv_*_batch
 * (kernels/mod.rs:858-902): n_tok vectors x_stride floats apart into n_tok
 * outputs y_stride floats apart (y_stride >= rows when n_tok > 1). The Q4
 * block sums of x are formed on the device. Host buffers; synchronous. */
int nnh_gemv_batch(const nnh_weight* w, const float* x, size_t x_stride, float* y, size_t y_stride, size_t n_tok,
                   int act);

/* model_argmax (model/forward.rs:989-1011) for a Q8_0/Q4 lm_head: the row of
 * the first largest logit of W x (ties to the lower row; NaN never wins, and
 * a NaN in row 0 keeps row 0). For a BF16 lm_head with rows % 4 == 0 and
 * cols % 8 == 0, gemv_bf16_argmax's running best (kernels/mod.rs:362-406):
 * ties to the lower row, NaN and -inf never taken, row 0 when none is.
 * Host x; synchronous. */
int nnh_model_argmax(const nnh_weight* w, const float* x, size_t* out_row, int act);

/* Device-resident form of nnh_model_argmax for f32 activations: x (cols
 * floats), logits (rows floats, written: W x) and work
 * (nnh_model_argmax_work_bytes(w) bytes) are device buffers, *out_row (a
 * device u64) receives the row; asynchronous on `stream`. For the matrices
 * of 12288 rows or more the first argmax stage runs inside the gemv (each
 * workgroup's best row), so only a one-workgroup reduction follows it.
 * Calls on different streams must not share `work`; a Q4 matrix under 12288
 * rows also uses the scratch of `stream` (as nnh_gemv_batch_dev). */
size_t nnh_model_argmax_work_bytes(const nnh_weight* w);
int nnh_model_argmax_dev(const nnh_weight* w, const float* x, float* logits, void* work, uint64_t* out_row,
                         void* stream);

/* Device-resident form of nnh_gemv_batch: x and y are device pointers, the
 * call is asynchronous on `stream` (a hipStream_t; NULL = the null stream).
 * The Q4 block sums / quantized activations / partial sums live in a
 * library-owned scratch buffer of that stream: calls on different streams
 * may overlap, as the reference's Model is shared by sessions on many
 * threads (lib.rs:36-41). A buffer that has to grow is replaced, and the old
 * one is kept until the process ends, so a call captured in a HIP graph stays
 * valid after larger calls; replays of graphs captured on the same stream
 * share that stream's scratch, so they must not overlap each other. */
int nnh_gemv_batch_dev(const nnh_weight* w, const float* x, size_t x_stride, float* y, size_t y_stride,
                       size_t n_tok, int act, void* stream);

/* The residual add and RMSNorm of the reference's forward (forward.rs:
 * 719-841, scalar.rs:232-292: v = x + r, then (v * scale) * gamma with
 * scale = 1 / sqrt(sum_sq(v) / cols + eps) in nncpu's order and rounding)
 * fused in front of one bit-exact f32 gemv: y = W ((v * scale) * gamma).
 * No counterpart in the reference, whose forward runs the norm and the
 * matmul as two calls; for a device-resident forward (one launch fewer per
 * norm in a decode step). r may be NULL (v = x). x_out and rec (either may
 * be NULL) receive v; neither may overlap x or r, which the call's
 * workgroups read while one of them writes. `normed` (cols floats) is
 * scratch the call may write the normed input to. All device pointers,
 * asynchronous on `stream`; the same bits as the norm followed by
 * nnh_gemv_batch_dev(..., NNH_ACT_F32). At most 16384 columns. */
int nnh_gemv_rmsnorm_dev(const nnh_weight* w, const float* x, const float* r, const float* gamma, float eps,
                         float* x_out, float* rec, float* normed, float* y, void* stream);

/* nnh_gemv_rmsnorm_dev with the activation mode named: NNH_ACT_F32 is that
 * call; NNH_ACT_I8 quantizes the normed input with nncpu's Q8_0 encoder
 * (quant.rs:31-60) and runs the int8 matmul on it, the same bits as the norm
 * followed by nnh_gemv_batch_dev(..., NNH_ACT_I8). No counterpart in the
 * reference (its forward quantizes inside each matmul call); for a
 * device-resident forward in the int8 mode. Rows of 97 to 256 blocks (3104
 * to 8192 columns) run the norm and the quantizer in the matmul's own
 * launch; other shapes run a norm kernel into `normed`, then the matmul. */
int nnh_gemv_rmsnorm_act_dev(const nnh_weight* w, int act, const float* x, const float* r, const float* gamma,
                             float eps, float* x_out, float* rec, float* normed, float* y, void* stream);

/* Device-resident argmax of model_argmax (model/forward.rs:1003-1011) over
 * n logits at v (device): the first largest value, NaN never winning and a
 * NaN at index 0 keeping 0. Writes the index to *out_row (device, u64);
 * asynchronous on `stream`. `work` is device memory of
 * nnh_argmax_work_bytes(n) bytes, owned by the caller (so the call
 * allocates nothing and can be captured in a HIP graph). */
size_t nnh_argmax_work_bytes(size_t n);
int nnh_argmax_dev(const float* v, size_t n, void* work, uint64_t* out_row, void* stream);

/* nnh_gemv_batch_dev for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): no
 * counterpart in the reference. Its scratch (Q4 block sums, quantized
 * activations, split-K partials) is one device array of
 * NNH_NOALLOC_SCRATCH_BYTES that the library holds on each GPU for the life
 * of the process; the call allocates nothing. Preconditions beyond
 * nnh_gemv_batch_dev's: nnh_init has run, and the weight's layouts for this
 * (act, n_tok) exist (nnh_weight_prepare, or an earlier nnh_gemv_batch_dev
 * call), else NNH_E_STATE; a call needing more scratch than the maximum
 * fails with NNH_E_INVALID (every call of up to 16 vectors fits at the
 * BASELINE shapes; large prefill batches may not). Every such call on one
 * GPU shares the array, whatever the stream: calls that overlap on one GPU
 * race (serialise them, e.g. on one stream). Nothing in the array needs to
 * start at zero: a call writes all it reads. */
#define NNH_NOALLOC_SCRATCH_BYTES (64u << 20)
int nnh_gemv_batch_dev_noalloc(const nnh_weight* w, const float* x, size_t x_stride, float* y, size_t y_stride,
                               size_t n_tok, int act, void* stream);

/* ---- int8 activation blocks (device memory, caller-owned) ----
 * An activation buffer holds n_tok vectors of `cols` values quantized with
 * nncpu's Q8_0 encoder, laid out as:
 *   int8_t   q[n_tok][cols]          the quants
 *   uint16_t s[n_tok][cols/32]       the BF16 block scales
 *   double   sx[n_tok][cols/32][2]   {bf16(s), s * sum(q of block)}, both exact
 *   float    sxT[2][cols/32][P]      the same two values block-major, for the
 *                                    MFMA GEMM (P = n_tok rounded up to 128)
 * at the offsets nnh_act_layout() reports (sxT follows sx); `bytes` is the
 * whole buffer. */
int nnh_act_layout(size_t cols, size_t n_tok, size_t* off_s, size_t* off_sx, size_t* bytes);

/* Quantize n_tok f32 vectors (device, x_stride apart) into `act`. */
int nnh_quantize_act_dev(const float* x, size_t x_stride, size_t cols, size_t n_tok, void* act, void* stream);

/* y (device, y_stride apart) = W x for activations already in `act`: the
 * int8 path without the quantization step. Batches of 4 or more vectors keep
 * split-K partial sums in the scratch of `stream` (as nnh_gemv_batch_dev). */
int nnh_gemv_i8_dev(const nnh_weight* w, const void* act, size_t n_tok, float* y, size_t y_stride, void* stream);

/* The same for either int8 mode (act = NNH_ACT_I8 or NNH_ACT_MXI8): the
 * buffer's layout (the MXI8 buffer is the NNH_ACT_I8 layout followed by the
 * GEMM's BF16 operands: xb = q 2^E in tiles of 256 tokens,
 * xb[T][cols/32][256][32] for T = n_tok rounded up to whole tiles, zero for
 * tokens past n_tok, the 16-byte chunk c of each 32-value row stored at
 * position c ^ ((t % 256 >> 2) & 3); and xl[P][nbp8][2] = the two BF16 limbs
 * of 2^E sum(q) per block, nbp8 = cols/32 rounded up to a multiple of 8),
 * the quantizer, and y = W x from a quantized buffer. The act-less
 * functions above are these with NNH_ACT_I8. No counterpart in the
 * reference (see NNH_ACT_MXI8). */
int nnh_act_layout_ex(int act, size_t cols, size_t n_tok, size_t* off_s, size_t* off_sx, size_t* bytes);
int nnh_quantize_act_ex_dev(int act, const float* x, size_t x_stride, size_t cols, size_t n_tok, void* buf,
                            void* stream);
int nnh_gemv_act_dev(const nnh_weight* w, int act, const void* buf, size_t n_tok, float* y, size_t y_stride,
                     void* stream);

/* Diagnostics: the exact int32 block dot products P[n][r][b] =
 * sum_k q_w[r, 32b+k] * q_x[n, 32b+k] (device output, rows*cols/32 per
 * vector), as the int8 path forms them. */
int nnh_block_dots_dev(const nnh_weight* w, const void* act, size_t n_tok, int32_t* P, void* stream);

/* Size the scratch of `stream` (and build the weight's layouts) for a call
 * (w, act, n_tok) ahead of time, so that such calls on `stream` allocate
 * nothing afterwards: for callers that capture them into a HIP graph, whose
 * first call would otherwise grow the stream's scratch inside the capture.
 * No counterpart in the reference, whose scratch is per session
 * (model/kv.rs:324-332). */
int nnh_stream_reserve(const nnh_weight* w, int act, size_t n_tok, void* stream);

/* Free the scratch the library holds for `stream` (its current buffer and
 * every outgrown one), after waiting for the work queued on it. For servers
 * that create a stream per session and end it: the scratch otherwise lives
 * until the process ends. Graphs captured on `stream` that used its scratch
 * must not be replayed afterwards; the next call on `stream` allocates
 * afresh. No counterpart in the reference. */
int nnh_stream_release(void* stream);

/* Block until all work the library queued on `stream` is done. */
int nnh_sync(void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NNCPU_HIP_H */
