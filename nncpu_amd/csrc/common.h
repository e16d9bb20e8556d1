// Shared device helpers and launcher declarations for libnncpu_hip.so.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace nnh {

// BF16 bits -> f32, exact (the BF16 bits are the high half of the f32;
// crates/nncpu/src/runtime.rs:10-13).
__device__ __forceinline__ float bf16f(uint32_t v) { return __uint_as_float(v << 16); }

// f32 -> BF16 bits, round to nearest even (runtime.rs:15-21).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Lane-exchange sums used by the reduction trees. `__shfl_xor` moves data
// through the LDS crossbar without touching LDS memory.
__device__ __forceinline__ float xor_get(float v, int mask) { return __shfl_xor(v, mask, 64); }
__device__ __forceinline__ double xor_get(double v, int mask) { return __shfl_xor(v, mask, 64); }

// f64 lane exchanges by DPP (a VALU modifier; no LDS traffic): each half of
// the double is moved with the same control. Controls used: 0xB1 quad_perm
// [1,0,3,2] (xor 1), 0x4E quad_perm [2,3,0,1] (xor 2), 0x141 row_half_mirror
// (lane i <-> 7-i within 8), 0x140 row_mirror (i <-> 15-i within 16).
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    int lo = __double2loint(v), hi = __double2hiint(v);
    lo = __builtin_amdgcn_update_dpp(0, lo, CTRL, 0xf, 0xf, false);
    hi = __builtin_amdgcn_update_dpp(0, hi, CTRL, 0xf, 0xf, false);
    return __hiloint2double(hi, lo);
}

// Sum over groups of L lanes (L in 2..64, a power of two); every lane of a
// group gets the group's sum. Fixed order, so the result is deterministic.
template <int L>
__device__ __forceinline__ double group_sum_f64(double v) {
    if (L >= 2) v += dpp_f64<0xB1>(v);
    if (L >= 4) v += dpp_f64<0x4E>(v);
    if (L >= 8) v += dpp_f64<0x141>(v);
    if (L >= 16) v += dpp_f64<0x140>(v);
    if (L >= 32) v += __shfl_xor(v, 16, 64);
    if (L >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// 16-byte load with the non-temporal hint: weights are streamed once per
// call and should not displace reused data (activations) in the caches.
typedef int nnh_v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 load_nt16(const void* p) {
    nnh_v4i v = __builtin_nontemporal_load((const nnh_v4i*)p);
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 load_nt16u(const void* p) {
    nnh_v4i v = __builtin_nontemporal_load((const nnh_v4i*)p);
    return make_uint4((unsigned)v.x, (unsigned)v.y, (unsigned)v.z, (unsigned)v.w);
}

// LDS pointer for __builtin_amdgcn_global_load_lds (global -> LDS, no
// staging registers): lane l's 16 bytes land at dst + 16 l, dst uniform.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt immediate with vmcnt = n (bits 3:0 and 15:14); expcnt and
// lgkmcnt at their maxima, so they do not wait. Direct-to-LDS loads count in
// vmcnt like any other vector memory load.
#define NNH_VMCNT(n) ((((n)&0xF) | (0x7 << 4) | (0xF << 8) | ((((n) >> 4) & 0x3) << 14)))
// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt at their maxima).
#define NNH_LGKMCNT0 (0xF | (0x7 << 4) | (0x3 << 14))

// s_waitcnt vmcnt(K) that is also a compiler memory barrier: every vector
// memory load issued before the K issued last has completed (loads complete
// in issue order), and no memory access moves across it. A kernel that
// issues direct-to-LDS copies and then K register loads waits for the copies
// alone with it; K must not exceed the number of load instructions issued
// after the copies. The base pointers of those K loads are passed in (a, b,
// c): loads through a __restrict__ argument are otherwise free to move
// across a "memory" clobber, and sunk below the wait they would leave copies
// in flight.
template <int K>
__device__ __forceinline__ void wait_vm_keep(const void* a = nullptr, const void* b = nullptr,
                                             const void* c = nullptr) {
    static_assert(K >= 0 && K <= 63, "vmcnt holds 0..63");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(K), "s"(a), "s"(b), "s"(c) : "memory");
}

// One 1 KB copy of the bytes [off, off + 1024) of a span of `len` bytes
// (a multiple of 16) to dst (uniform); lanes past the end repeat the span's
// last 16 bytes. Issued as asm: for the builtin the compiler cannot tell
// the copy's LDS destination from any later LDS read and waits for every
// copy before each read, which would undo the staging (the waits here are
// explicit instead).
__device__ __forceinline__ void copy_1k(const void* span, size_t len, size_t off, unsigned char* dst, int lane) {
    const size_t o = min(off + lane * 16, len - 16);
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"((const unsigned char*)span + o),
                 "{m0}"((uint32_t)(uintptr_t)dst)
                 : "memory");
}

// Compute units of the current device (kernels_misc.hip).
int cu_count();

inline int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

// ---- launchers (defined beside their kernels) -------------------------------

// Upload-time relayouts for the bit-exact f32 path (kernels_f32.hip).
// `v2`: the 8-lane layout and kernel (tall matrices, x of one token within
// F32_V2_MAX_LDS bytes); f32_quant_bytes is the size of the quant layout
// either way.
constexpr int F32_V2_MAX_LDS = 64 * 1024;
size_t f32_quant_bytes(int dtype, int rows, int nb, bool v2);
void launch_relayout_f32(int dtype, const uint8_t* raw_qs, const uint16_t* raw_scales, uint8_t* fq, uint16_t* fs,
                         int rows, int nb, int nbp, bool v2, hipStream_t st);
// Q4 block sums of n_tok vectors (kernels/scalar.rs:355-359 tree).
void launch_block_sums(const float* x, size_t x_stride, int nb, int n_tok, float* xsum, hipStream_t st);
// Bit-exact f32 gemv for n_tok <= 16 vectors; for Q4, xsum is scratch of
// n_tok * nb floats (the block sums of x).
// One vector through the 8-lane (tall) kernel, y written and each
// workgroup's largest argmax key into part[0..f32_v2_parts(rows)).
int f32_v2_parts(int rows);
void launch_gemv_f32_v2_argmax(int dtype, const uint8_t* fq, const uint16_t* fs, const uint16_t* biases,
                               const float* x, float* xsum, int rows, int nb, int nbp, float* y, uint64_t* part,
                               hipStream_t st);
// The residual add and RMSNorm that a one-vector gemv can run on its input
// first (nnh_gemv_rmsnorm_dev, nnh_gemv_rmsnorm_act_dev): v = x + r (r NULL:
// v = x), then the gemv's input is (v * rms(v)) * gamma. Workgroup 0 writes
// v to x_out and rec (either may be NULL); x_out must not overlap x, which
// other workgroups may still be reading.
struct NormIn {
    const float* x;
    const float* r;
    const float* gamma;
    float* x_out;
    float* rec;
    float eps;
};

// One vector with the fused residual add and RMSNorm: the streamed or tall
// kernel with the norm in its prologue; false (nothing launched) when
// neither applies (the caller then runs launch_rmsnorm_vec, at most 16384
// columns, and the plain gemv).
bool launch_gemv_f32_norm(int dtype, const uint8_t* fq, const uint16_t* fs, const uint16_t* biases,
                          const NormIn& nrm, int rows, int nb, int nbp, float* y, bool v2, hipStream_t st);
void launch_rmsnorm_vec(const NormIn& nrm, int cols, float* out, hipStream_t st);
void launch_gemv_f32(int dtype, const uint8_t* fq, const uint16_t* fs, const uint16_t* biases, const float* x,
                     size_t x_stride, float* xsum, int rows, int nb, int nbp, int n_tok, float* y,
                     size_t y_stride, bool v2, hipStream_t st);

// int8 path (kernels_i8.hip).
void launch_quantize_act(const float* x, size_t x_stride, int cols, int n_tok, int8_t* q, uint16_t* s, double* sx,
                         float* sxT, int tok_pad, hipStream_t st);
void launch_pack_sb(const uint16_t* sc, const uint16_t* bi, uint32_t* sb, size_t n, hipStream_t st);
void launch_gemv_i8(int dtype, const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const uint32_t* sb,
                    const int8_t* aq, const double* asx, int rows, int nb, int n_tok, float* y, size_t y_stride,
                    hipStream_t st);
// One vector with the residual add, RMSNorm and Q8_0 quantizer fused into
// the int8 GEMV's prologue (same bits as launch_rmsnorm_vec, the quantizer
// and launch_gemv_i8 in turn); false (nothing launched) when the shape or
// alignment does not fit it (rows of 97 .. 256 blocks, 16-byte aligned
// vectors, Q4 with its packed scale-and-bias words).
bool launch_gemv_i8_norm(int dtype, const uint8_t* qs, const uint16_t* scales, const uint32_t* sb,
                         const NormIn& nrm, int rows, int nb, float* y, hipStream_t st);
// One f32 vector quantized with nncpu's Q8_0 encoder in the int8 GEMV's
// prologue (same bits as the quantizer then launch_gemv_i8); false (nothing
// launched) where it measured slower than the two launches or the shape or
// alignment does not fit it (rows of 97 .. 384 blocks, except tall Q8
// matrices of rows that are not whole 64-block groups; x 16-byte aligned;
// Q4 with its packed scale-and-bias words).
bool launch_gemv_i8_qx(int dtype, const uint8_t* qs, const uint16_t* scales, const uint32_t* sb, const float* x,
                       int rows, int nb, float* y, hipStream_t st);
// f32 -> Q8_0 / Q4 split layout on the device (kernels_encode.hip).
void launch_encode(int dtype, const float* w, size_t n, uint8_t* qs, uint16_t* sc, uint16_t* bi, hipStream_t st);
// BF16 weights (kernels_bf16.hip): the reference's kernel by shape.
enum { BF16_PATH_F64 = 0, BF16_PATH_QUAD = 1, BF16_PATH_ROW8 = 2, BF16_PATH_ROW32 = 3 };
int bf16_path(size_t rows, size_t cols);
size_t bf16_layout_bytes(int path, size_t rows, size_t cols);  // 0 for the f64 path
void launch_relayout_bf16(int path, const uint16_t* raw, uint16_t* bl, int rows, int cols, hipStream_t st);
void launch_gemv_bf16(int path, const uint16_t* raw, const uint16_t* bl, int rows, int cols, const float* x,
                      size_t x_stride, int n_tok, float* y, size_t y_stride, hipStream_t st);
void launch_encode_bf16(const float* w, size_t n, uint16_t* out, hipStream_t st);
// GGUF tensor blocks -> f32 (kernels_gguf.hip): bytes and values per block
// of a decodable ggml type; the decode itself (n a whole number of blocks).
bool ggml_block(uint32_t type, size_t* bytes, size_t* per);
void launch_dequantize(uint32_t type, const uint8_t* src, size_t n, float* dst, hipStream_t st);
// int8 MFMA GEMM for many vectors (kernels_gemm.hip).
int gemm_rows_pad(int rows);
int gemm_tok_pad(int n_tok);
void launch_gemm_scales(const uint16_t* sc, const uint16_t* bi, float* swT, int rows, int nb, hipStream_t st);
size_t gemm_workspace_bytes(int rows, int nb, int n_tok);  // split-K partials; 0 if unsplit
// int8 MFMA matmul for 5..16 vectors (kernels_skinny.hip).
size_t skinny_workspace_bytes(int rows, int nb);  // K-split partials; 0 if unsplit
void launch_skinny_i8(int dtype, const uint8_t* qs, const float* swT, const int8_t* aq, const float* sxT, int rows,
                      int nb, int n_tok, float* y, size_t y_stride, double* ws, hipStream_t st);
void launch_gemm_i8(int dtype, const uint8_t* qs, const float* swT, const int8_t* aq, const float* sxT, int rows,
                    int nb, int n_tok, float* y, size_t y_stride, double* ws, hipStream_t st);
void launch_block_dots(int dtype, const uint8_t* qs, const int8_t* aq, int rows, int nb, int n_tok, int32_t* P,
                       hipStream_t st);
// MX int8 path (kernels_mx.hip): power-of-two activation scales and the BF16
// MFMA GEMM. nbp8 = nb rounded up to whole 8-block groups.
int mx_nbp8(int nb);
void launch_quantize_mx(const float* x, size_t x_stride, int cols, int n_tok, int8_t* q, uint16_t* s, double* sx,
                        float* sxT, int tok_pad, uint16_t* xb, uint16_t* xl, hipStream_t st);
size_t mx_bias_bytes(int rows, int nb);    // Q4 biases twice, rows padded
int mx_xl_tok(int n_tok);                  // GEMM token tiles' worth of tokens
size_t mx_xl_bytes(int n_tok, int nb);     // X limbs, tokens padded to mx_xl_tok
void launch_mx_bias(const uint16_t* bi, int rows, int nb, uint16_t* wbi, hipStream_t st);
size_t gemm_mx_workspace_bytes(int rows, int nb, int n_tok);  // f32 partial tiles
void launch_gemm_mx(int dtype, const uint8_t* qs, const float* swT, const uint16_t* wbi, const uint16_t* xb,
                    const uint16_t* xl, int rows, int nb, int n_tok, float* y, size_t y_stride, float* ws,
                    hipStream_t st);

// argmax over n logits (kernels_misc.hip); partial holds 2*ceil(n/2048) words.
// The argmax key of value v at row idx: an order-preserving image of v in
// the high word (-0 folded onto +0, which compare equal), the complement of
// the index in the low word, so the largest key is the largest value at its
// lowest row; NaN gets key 0.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    if (!(v == v)) return 0;
    if (v == 0.0f) v = 0.0f;
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - idx);
}

// The largest key of each part -> the row (v: the values, read for row 0's
// NaN rule in mode 0).
void launch_argmax_final(const float* v, const uint64_t* partial, int nparts, uint64_t* out, hipStream_t st,
                         int mode);
// mode 0: the first largest value, a NaN in row 0 keeping row 0
// (forward.rs:1003-1011); mode 1: the BF16 4-row kernel's running best from
// -inf (scalar.rs:612-628): NaN and -inf never taken, none taken gives 0.
void launch_argmax(const float* v, size_t n, uint64_t* partial, uint64_t* out, hipStream_t st, int mode = 0);
size_t argmax_partial_words(size_t n);

}  // namespace nnh
