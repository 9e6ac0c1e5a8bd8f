/*
 * w4a16.h -- C ABI of the MI355X (gfx950) INT4-weight / bf16-activation linear.
 *
 * Plain pointers and sizes only.  Every device pointer is borrowed: the caller
 * owns and allocates all buffers (inputs, output and workspace), so a call never
 * allocates and can be captured into a HIP graph.  Work is enqueued on `stream`
 * (a hipStream_t passed as void*; NULL means the default stream).  No exception
 * crosses this boundary: every entry point returns a W4A16_* status code.
 *
 * Data layout (the reference format, engine/kernels/quant.py:81-119):
 *   x       bf16  [M, K]     row stride ldx elements, unit column stride
 *   packed  int8  [K/2, N]   row stride ldp bytes; byte (i, n) holds q[2i, n] in
 *                            bits 7..4 and q[2i+1, n] in bits 3..0, both 4-bit
 *                            two's complement
 *   scale   fp32  [K/g, N]   row stride lds elements, g = group_size
 *   y       bf16  [M, N]     row stride ldy elements
 */
#ifndef W4A16_H_
#define W4A16_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A16_ABI_VERSION 7

/* Most problems one grouped call accepts. */
#define W4A16_MAX_PROBLEMS 16

/* Status codes. */
#define W4A16_OK 0
#define W4A16_ERR_NULL 1        /* a required pointer is NULL */
#define W4A16_ERR_SHAPE 2       /* negative size, leading dimension smaller than the row, or bad count */
#define W4A16_ERR_K_GROUP 3     /* K not a multiple of group_size, or odd */
#define W4A16_ERR_GROUP_SIZE 4  /* group_size unsupported (linear: must be 128) */
#define W4A16_ERR_WORKSPACE 5   /* workspace NULL or smaller than w4a16_workspace_size() */
#define W4A16_ERR_LAUNCH 6      /* a HIP launch reported an error */
#define W4A16_ERR_DTYPE 7       /* unknown dtype code */
#define W4A16_ERR_TOO_LARGE 8   /* problem exceeds what the entry point supports (w4a16_bf16_gemv: M > 16;
                                   decode-sized M whose split-K partials, nsplit * M * N * 4 bytes, reach 4 GB) */
#define W4A16_ERR_CAPTURING 9   /* the stream is capturing a graph and the call needs eager work first
                                   (w4a16_linear_noalloc before its scratch is set up; w4a16_noalloc_status) */

/* Bits of a workspace's status word (see w4a16_status_offset). */
#define W4A16_STATUS_SPLITK_TIMEOUT 1u  /* a decode split-K finisher gave up polling: its outputs are NaN and
                                           the workspace's slot half may hold stale partials (zero it again) */

/* dtype codes for w4a16_dequant. */
#define W4A16_DTYPE_F32 0
#define W4A16_DTYPE_BF16 1

/*
 * One projection y[M, N] = x[M, K] @ W[K, N] of a grouped call.  Layouts as
 * for w4a16_linear; every problem has its own M (a set of MoE experts with
 * their own token counts) or the same (q/k/v, gate/up).
 */
typedef struct w4a16_problem {
  const void* x;        /* bf16 [M, K] */
  int64_t ldx;
  const int8_t* packed; /* [K/2, N] */
  int64_t ldp;
  const float* scale;   /* [K/128, N] */
  int64_t lds;
  void* y;              /* bf16 [M, N] */
  int64_t ldy;
  int M;
  int N;
  int K;
} w4a16_problem;

/* Version of this ABI (W4A16_ABI_VERSION of the build). */
int w4a16_abi_version(void);

/* Static description of a status code. */
const char* w4a16_error_string(int code);

/*
 * Bytes of device workspace w4a16_linear needs for an (M, N, K) call; 0 means
 * the call needs none.  The size covers any operand alignment (activations
 * whose rows are not 16-byte aligned run M > 32 through the decode kernel 32
 * rows at a time, which can need more than the GEMM).  A workspace of W bytes is used in two halves: the
 * lower half holds the decode kernels' split-K partial slots, which must be
 * zero before the first call that uses the buffer and are left at zero by
 * every completed call; the upper half is GEMM scratch.  So: zero a buffer
 * once when it is allocated, pass its full size on every call, and replace it
 * by a new zeroed buffer to grow it.  Calls that share a workspace must be
 * ordered (same stream).  The last aligned 32-bit word of the workspace is its
 * status word (w4a16_status_offset).  Replaces no reference entry point: the
 * reference kernel needs no workspace (engine/kernels/quant.py:270-280
 * allocates only the output).
 */
int w4a16_workspace_size(int M, int N, int K, int group_size, size_t* bytes);

/*
 * y[M, N] = x[M, K] @ dequant(packed, scale)[K, N], bf16 output, fp32
 * accumulation, per-group partial products scaled in fp32.
 *
 * Replaces the device branch of int4_matmul (engine/kernels/quant.py:267-281),
 * i.e. the launch of _int4_matmul_kernel (engine/kernels/quant.py:159-240), and
 * with it the whole of _Int4Weight.fused_linear (engine/quantize.py:64-73)
 * once the caller has flattened x to [M, K].
 *
 * group_size must be 128 (the reference asserts the same,
 * engine/kernels/quant.py:267).  K must be a multiple of 128.  M == 0 or
 * N == 0 is a no-op; K == 0 writes zeros.  M <= 32 runs the bandwidth-bound
 * decode kernel, M > 64 the MFMA GEMM; 32 < M <= 64 takes the decode kernel
 * when N/64 * K/1024 <= 1024 (its workgroup count), else the GEMM.
 */
int w4a16_linear(const void* x, int64_t ldx,
                 const int8_t* packed, int64_t ldp,
                 const float* scale, int64_t lds,
                 void* y, int64_t ldy,
                 int M, int N, int K, int group_size,
                 void* workspace, size_t workspace_bytes,
                 void* stream);

/*
 * w4a16_linear without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture with no allocator,
 * tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference.  Same arguments (minus the workspace), arithmetic, results
 * and status codes as w4a16_linear.  Its scratch is a fixed 96 MiB array in
 * the library's own device memory, one per GPU, held until the process ends.
 * The first call on a device that needs the scratch sets it up: it looks up
 * the array's address, zeroes it on `stream` and waits for that fill.  That
 * first call must be eager: made while `stream` is capturing a graph it
 * returns W4A16_ERR_CAPTURING and launches nothing (make one eager call, or
 * call w4a16_noalloc_status, on the device first).  Calls whose split-K
 * scratch (w4a16_workspace_size) exceeds 96 MiB return W4A16_ERR_TOO_LARGE
 * before anything is launched.  The call itself never allocates.  Every call
 * on one GPU shares that GPU's array, which keeps the last call's contents:
 * calls that overlap on one GPU (other streams or threads) race, so order
 * them.  A split-K give-up (W4A16_STATUS_SPLITK_TIMEOUT) is reported and
 * cleared by w4a16_noalloc_status.
 */
int w4a16_linear_noalloc(const void* x, int64_t ldx,
                         const int8_t* packed, int64_t ldp,
                         const float* scale, int64_t lds,
                         void* y, int64_t ldy,
                         int M, int N, int K, int group_size,
                         void* stream);

/*
 * Status word of the current device's no-alloc scratch (W4A16_STATUS_*), for
 * w4a16_linear_noalloc as w4a16_status_offset is for a workspace.  No
 * counterpart in the reference, whose kernel has no cross-workgroup protocol;
 * it is for the callers of w4a16_linear_noalloc, which cannot allocate.
 * Synchronises `stream`, reads the word and, when it is set (a finisher gave
 * up and late partials may sit in the slots), zeroes the whole scratch on
 * `stream` and waits for it, so later calls start from empty slots.  Sets the
 * scratch up if no call has yet.  Refused while `stream` is capturing
 * (W4A16_ERR_CAPTURING).  Allocates nothing; do not overlap it with
 * w4a16_linear_noalloc calls on the same GPU.
 */
int w4a16_noalloc_status(void* stream, uint32_t* status);

/*
 * Identity of the graph capture `stream` is in: a non-zero id unique to that
 * capture, or 0 when the stream is not capturing.  No counterpart in the
 * reference.  Host bookkeeping for callers that keep one workspace per
 * stream: a workspace first allocated inside a capture is zeroed by a fill
 * that only that graph holds, so every other capture that uses it must record
 * a fill of its own (once per capture) for its replays not to depend on which
 * graph has replayed first.
 */
int w4a16_capture_id(void* stream, unsigned long long* id);

/*
 * Several independent projections: up to W4A16_MAX_PROBLEMS problems, each
 * with its own M, activations, weights and output (problems may share x, e.g.
 * q/k/v or gate/up of a decoder block).  Problems that take the decode
 * kernel (see w4a16_linear) run in one decode launch, the rest in one GEMM
 * launch.  Same arithmetic and status codes as
 * w4a16_linear; the workspace must be at least w4a16_workspace_size_grouped()
 * for the same table.
 *
 * No counterpart in the reference, which calls int4_matmul once per projection
 * (engine/llama_attention.py:83-85, engine/llama_mlp.py:30-33) and once per
 * active expert and projection (engine/llama_moe.py:90-105).  It is the
 * fused-projection path for those call sites: one launch streams all the
 * listed weights.
 */
int w4a16_linear_grouped(const w4a16_problem* problems, int count, int group_size,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Byte offset of the status word inside a workspace of workspace_bytes bytes
 * (the last aligned 32-bit word; workspaces under 256 bytes have none and
 * return W4A16_ERR_WORKSPACE).  It is zero as allocated; a decode split-K
 * finisher that exhausts its poll budget ORs W4A16_STATUS_SPLITK_TIMEOUT into
 * it (and writes NaN outputs).  Read it after synchronising the stream; when
 * it is set, zero the whole workspace before its next use.  No counterpart in
 * the reference, whose kernel has no cross-workgroup protocol.
 */
int w4a16_status_offset(size_t workspace_bytes, size_t* offset);

/*
 * Poll budget of the decode split-K finisher for later calls in this process
 * (default 2^20 rounds; returns the previous value).  For tests of the
 * give-up path: a budget of 0 makes a finisher give up as soon as one of its
 * slots is still empty, so every kernel still ends normally.
 */
uint32_t w4a16_debug_set_spin_limit(uint32_t polls);

/* Workspace bytes w4a16_linear_grouped needs for this problem table. */
int w4a16_workspace_size_grouped(const w4a16_problem* problems, int count, int group_size, size_t* bytes);

/*
 * SwiGLU gate/up pair: h[M, N] = silu(x @ Wg) * (x @ Wu), silu(v) = v *
 * sigmoid(v), with Wg and Wu INT4 weights of the same shape in the layout
 * above (their own leading dimensions), bf16 h with row stride ldh.
 *
 * Replaces `silu(linear(x, gate)) * linear(x, up)` of the reference MLP
 * (engine/llama_mlp.py:30-32, engine/llama_moe.py:44), i.e. two int4_matmul
 * launches plus two elementwise kernels.  Decode-sized M (as in w4a16_linear) runs one decode launch that
 * streams both weights and applies the epilogue to the fp32 sums (the
 * reference rounds gate and up to bf16 first; results agree to bf16 rounding).
 * GEMM-sized M runs the row sums and then one pair GEMM launch whose
 * workgroups compute matching gate and up tiles and store silu(g) * u from
 * the fp32 sums.  Operands the pair GEMM cannot take (N not a multiple of
 * 128, fewer than 256 tiles, unaligned rows) go through a grouped GEMM (gate
 * into h, up into workspace) and one elementwise pass.  Status codes,
 * group_size and workspace rules as w4a16_linear, with
 * w4a16_workspace_size_swiglu() in place of w4a16_workspace_size().
 */
int w4a16_swiglu(const void* x, int64_t ldx,
                 const int8_t* gate_packed, int64_t gate_ldp, const float* gate_scale, int64_t gate_lds,
                 const int8_t* up_packed, int64_t up_ldp, const float* up_scale, int64_t up_lds,
                 void* h, int64_t ldh,
                 int M, int N, int K, int group_size,
                 void* workspace, size_t workspace_bytes,
                 void* stream);

/* Workspace bytes w4a16_swiglu needs for an (M, N, K) call (0: none). */
int w4a16_workspace_size_swiglu(int M, int N, int K, int group_size, size_t* bytes);

/*
 * Dense bf16 GEMV for decode: y[m, n] = sum_k x[m, k] * w[n, k] with w in
 * Linear layout [N, K] (row stride ldw elements), fp32 accumulation, bf16
 * output; M <= 16.  x and w must be 16-byte aligned with K, ldx and ldw
 * multiples of 8.  No workspace.
 *
 * Replaces the decode case of `logits = x @ self.w.lm_head.T`
 * (engine/llama_model.py:148, engine/llama_moe_model.py:206), whose bf16
 * lm_head the reference leaves unquantized (engine/quantize.py:23).  Returns
 * W4A16_ERR_TOO_LARGE for M > 16 (callers use a library GEMM there).
 */
int w4a16_bf16_gemv(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
                    int M, int N, int K, void* stream);

/*
 * out[K, N] = q[K, N] * scale[k / group_size, n]  in fp32 (out_dtype
 * W4A16_DTYPE_F32), or with scale and product both rounded to bf16
 * (W4A16_DTYPE_BF16), i.e. dequantize_weight_int4(packed, scale.to(dtype))
 * of engine/kernels/quant.py:122-156 for dtype float32 / bfloat16.  Any
 * group_size > 0 dividing K.  Row stride of out: ldo elements.
 */
int w4a16_dequant(const int8_t* packed, int64_t ldp,
                  const float* scale, int64_t lds,
                  void* out, int64_t ldo, int out_dtype,
                  int K, int N, int group_size,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_H_ */
