/* xrmm: MI355X (gfx950) MatMulNBits / MatMulNBitsQkv / MatMulNBitsMlp, QMoE,
 * GatherBlockQuantized and MatMulBnb4.
 *
 * C ABI of libxrmm.so. Plain pointers and sizes only. Every entry point
 * returns XRMM_OK or an error class and leaves a thread-local message for
 * xrmm_last_error().
 *
 * Error classes mirror the reference's two exception types
 * (kernels/_shared/extended/planner.cpp, vulkan.cpp:105,115):
 *   XRMM_EINVAL  <- std::invalid_argument (contract, shape, attribute problems)
 *   XRMM_EDEVICE <- std::runtime_error    (device, timeout, GPU-side failures)
 *
 * dtype codes follow the order of xrgpu::operators::DType
 * (runtime/include/xrgpu/operators.h:9).
 */
#ifndef XRMM_H
#define XRMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  XRMM_OK = 0,
  XRMM_EINVAL = 1,
  XRMM_EDEVICE = 2,
};

/* runtime/include/xrgpu/operators.h:9 enum class DType */
enum {
  XRMM_F32 = 0,
  XRMM_F16 = 1,
  XRMM_I32 = 2,
  XRMM_U32 = 3,
  XRMM_I16 = 4,
  XRMM_I8 = 5,
  XRMM_U8 = 6,
  XRMM_I64 = 7,
  XRMM_BOOL = 8,
  XRMM_UNSPECIFIED = 9,
};

/* Fused activation kinds of MatMulNBitsMlp; the codes are those of
 * activation_lower (kernels/_shared/extended/complex_plan.cpp:55). */
enum {
  XRMM_ACT_NONE = 0,
  XRMM_ACT_RELU = 1,
  XRMM_ACT_SILU = 2,
  XRMM_ACT_GELU = 3,
  XRMM_ACT_TANH = 4,
  XRMM_ACT_SIGMOID = 5,
  XRMM_ACT_SWIGLU = 6, /* passes the gate value through, as the shader does */
};

/* Message of the last failed call on this thread ("" if none). */
const char* xrmm_last_error(void);

/* Library version string. */
const char* xrmm_version(void);

/* ---------------------------------------------------------------------------
 * Zero-copy entry points: every tensor pointer is a DEVICE pointer of the
 * current HIP device, contiguous row-major; `stream` is a hipStream_t (NULL =
 * the null stream). They enqueue work and return without synchronising.
 *
 * Zero points (`zp_dtype`):
 *   XRMM_UNSPECIFIED  absent: z = 2^(bits-1)
 *   XRMM_F32/XRMM_F16 float zero points [N, ceil(K/block_size)] (reference T3)
 *   XRMM_U8           packed uint8 [N, ceil(ceil(K/block_size)*bits/8)],
 *                     low-first (ONNX Runtime layout; an extension)
 * `dtype` is T1 (XRMM_F32 or XRMM_F16): the type of A, scales, bias, outputs.
 * ------------------------------------------------------------------------- */

/* com.microsoft.MatMulNBits, opcode 1025.
 * Replaces the serial packedMatmul path of
 * kernels/_shared/extended/shaders/complex_kernel.glsl:80,83 as planned by
 * kernels/_shared/extended/complex_plan.cpp:117-120 (inputs
 * aT,bT,scalesT,zeroPointsT?,biasT?; output yT = aT.shape[:-1]+[N]).
 * A [M,K], B [N,kb,blob] u8, scales [N,kb], bias [N] or NULL, Y [M,N]. */
int xrmm_matmul_nbits(const void* A, const void* B, const void* scales, const void* zero_points,
                      int32_t zp_dtype, const void* bias, void* Y, int64_t M, int64_t K,
                      int64_t N, int32_t bits, int32_t block_size, int32_t dtype, void* stream);

/* xrmm_matmul_nbits with a caller's workspace, for geometries whose output
 * tiles leave compute units idle (more than 16 rows with few columns or few
 * rows; the Llama-style down projection K = 14336, N = 4096 has 64 column
 * tiles on the thin GEMM at 17..64 rows and 32 tiles on the 128 x 128 GEMM
 * at 65..127 rows, for 256 CUs): the K range is split over workgroups, each
 * split writes a float32 partial tile to the workspace and the last split of
 * a tile adds them in split order (deterministic). No counterpart in the
 * reference (one serial loop, complex_kernel.glsl:83); same results as
 * xrmm_matmul_nbits within the float16 bar.
 * The workspace also carries the float32-arithmetic MFMA GEMM that runs
 * more than 16 rows of float32 activations, or of float16 activations with
 * 2- or 8-bit codes (from 12 rows for weight matrices of 2^24 codes or more,
 * from 5 rows for 2^25 or more; "gemm_f32_mfma"; without a workspace those calls take
 * the float32-arithmetic GEMV): its prepared rows (binary16 hi / lo terms of
 * float32 activations, block sums for float zero points) and split partials;
 * same results as xrmm_matmul_nbits within the float32 bar (float32
 * activations) or within one binary16 rounding of float32 arithmetic
 * (float16).
 * xrmm_matmul_nbits_workspace_bytes gives the bytes (0: neither applies,
 * and the call runs like xrmm_matmul_nbits). The workspace is 256-byte
 * aligned; its first 4096 bytes (per-tile arrival counters) are zero before
 * its first use and every call leaves them zero, so one workspace serves
 * consecutive calls of any shape on a stream. Calls that may overlap
 * (different streams) need different workspaces. */
int64_t xrmm_matmul_nbits_workspace_bytes(int64_t M, int64_t K, int64_t N, int32_t bits,
                                          int32_t block_size, int32_t dtype);
int xrmm_matmul_nbits_ws(const void* A, const void* B, const void* scales, const void* zero_points,
                         int32_t zp_dtype, const void* bias, void* Y, int64_t M, int64_t K, int64_t N,
                         int32_t bits, int32_t block_size, int32_t dtype, void* workspace,
                         int64_t workspace_bytes, void* stream);

/* Offline weight prepack for the prefill GEMM. The reference has no
 * counterpart in code; it is the "prepare = upload / prepack" step of its
 * Operator lifecycle (kernels/_shared/extended/vulkan.cpp:119) for callers
 * that hold their weights on the device. The 4-bit codes of B [N,kb,blob]
 * are rewritten K-step-major ([ceil(kb*block_size/64)][N][32 bytes], a K step
 * being 64 codes) with the codes of each 32-bit word reordered so that the
 * GEMM dequantises in natural k order; scales and zero points keep their
 * layout. xrmm_prepacked_bytes returns the packed size, 0 when the geometry
 * has none (bits other than 4, or columns not of whole 32-code chunks).
 * Both pointers 16-byte aligned. */
int64_t xrmm_prepacked_bytes(int64_t N, int64_t K, int32_t bits, int32_t block_size);
int xrmm_prepack_weights(const void* B, void* packed, int64_t N, int64_t K, int32_t bits,
                         int32_t block_size, void* stream);

/* xrmm_matmul_nbits with B prepacked by xrmm_prepack_weights (float16 A and
 * outputs, 4-bit codes, power-of-two block_size >= 16, K a multiple of 8,
 * 16-byte aligned tensors; other geometries return XRMM_EINVAL). Runs the
 * 256 x 256 prefill GEMM for every M. The request lifecycle (xrmm_prepare)
 * prepacks by itself for MatMulNBits requests that reach that GEMM. */
int xrmm_matmul_nbits_prepacked(const void* A, const void* packed, const void* scales,
                                const void* zero_points, int32_t zp_dtype, const void* bias, void* Y,
                                int64_t M, int64_t K, int64_t N, int32_t bits, int32_t block_size,
                                int32_t dtype, void* stream);

/* com.microsoft.MatMulNBitsQkv, opcode 1028 (complex_kernel.glsl:81,83;
 * complex_plan.cpp:37,119). x = RMSNorm(A + skip) * norm_scale (eps), then
 * Q = x Wq^T [M,Nq], K = x Wk^T [M,Nkv], V = x Wv^T [M,Nkv]; residual
 * (A + skip, [M,K]) is written when non-NULL. skip may be NULL. The three
 * zero-point pointers are an extension (NULL = implicit midpoint) and share
 * `zp_dtype`. */
int xrmm_matmul_nbits_qkv(const void* A, const void* skip, const void* norm_scale,
                          const void* q_B, const void* q_scales, const void* q_zero_points,
                          const void* k_B, const void* k_scales, const void* k_zero_points,
                          const void* v_B, const void* v_scales, const void* v_zero_points,
                          int32_t zp_dtype, void* Q, void* Kout, void* V, void* residual,
                          int64_t M, int64_t K, int64_t Nq, int64_t Nkv, int32_t bits,
                          int32_t block_size, float epsilon, int32_t dtype, void* stream);

/* com.microsoft.MatMulNBitsMlp, opcode 1027 (complex_kernel.glsl:39-47,81,83;
 * complex_plan.cpp:36,55,118). x = A + skip, RMS-normalised by norm_scale when
 * that is non-NULL; Y = act(x Wg^T + gate_bias) * (x Wu^T + up_bias) [M,N];
 * residual (A + skip) is written when non-NULL. Zero points are an extension
 * (NULL = implicit midpoint). */
int xrmm_matmul_nbits_mlp(const void* A, const void* skip, const void* norm_scale,
                          const void* gate_B, const void* gate_scales, const void* gate_zero_points,
                          const void* gate_bias, const void* up_B, const void* up_scales,
                          const void* up_zero_points, const void* up_bias, int32_t zp_dtype,
                          void* Y, void* residual, int64_t M, int64_t K, int64_t N, int32_t bits,
                          int32_t block_size, float epsilon, int32_t activation, int32_t dtype,
                          void* stream);

/* xrmm_matmul_nbits_qkv / xrmm_matmul_nbits_mlp with a caller's workspace for
 * the prefill GEMMs (more than 16 rows): a prologue kernel computes
 * x = RMSNorm(A + skip) * norm_scale (or A + skip) once per row into the
 * workspace as binary16, rounded after the normalisation (packedInput,
 * complex_kernel.glsl:81), and writes the residual; the GEMM then reads x
 * (from 128 rows with enough tiles: the 256 x 256 prefill pipeline, the three
 * Qkv projections on one grid, Mlp gate and up columns interleaved with
 * act(g) * u in the epilogue). xrmm_matmul_nbits_fused_workspace_bytes gives
 * the bytes (op: 1 Qkv, 2 Mlp; N = Nq for Qkv; 0 = none needed, the call runs
 * like the workspace-free entry point). The workspace is 256-byte aligned;
 * nothing in it needs clearing; calls that may overlap need different
 * workspaces. No counterpart in the reference (one serial loop); same results
 * as the entry points above within the float16 bar. */
int64_t xrmm_matmul_nbits_fused_workspace_bytes(int32_t op, int64_t M, int64_t K, int64_t N, int64_t Nkv,
                                                int32_t bits, int32_t block_size, int32_t dtype, int32_t has_skip,
                                                int32_t has_norm_scale);
int xrmm_matmul_nbits_qkv_ws(const void* A, const void* skip, const void* norm_scale,
                             const void* q_B, const void* q_scales, const void* q_zero_points,
                             const void* k_B, const void* k_scales, const void* k_zero_points,
                             const void* v_B, const void* v_scales, const void* v_zero_points,
                             int32_t zp_dtype, void* Q, void* Kout, void* V, void* residual,
                             int64_t M, int64_t K, int64_t Nq, int64_t Nkv, int32_t bits,
                             int32_t block_size, float epsilon, int32_t dtype, void* workspace,
                             int64_t workspace_bytes, void* stream);
int xrmm_matmul_nbits_mlp_ws(const void* A, const void* skip, const void* norm_scale,
                             const void* gate_B, const void* gate_scales, const void* gate_zero_points,
                             const void* gate_bias, const void* up_B, const void* up_scales,
                             const void* up_zero_points, const void* up_bias, int32_t zp_dtype, void* Y,
                             void* residual, int64_t M, int64_t K, int64_t N, int32_t bits,
                             int32_t block_size, float epsilon, int32_t activation, int32_t dtype,
                             void* workspace, int64_t workspace_bytes, void* stream);

/* Dequantized weights W [N,K] (nbitWeight, complex_kernel.glsl:80) in
 * `out_dtype`: XRMM_F32 gives the reference value (float(code) - z) * scale;
 * XRMM_F16 gives that value rounded once to binary16, produced by the same
 * device dequantisation routine the fp16 GEMV/GEMM kernels use. `scale_dtype`
 * is the dtype of `scales`. The reference has no standalone dequantisation
 * entry; this one exposes the kernels' weight staging for bit-exact checks. */
int xrmm_dequantize(const void* B, const void* scales, const void* zero_points, int32_t zp_dtype,
                    void* W, int64_t N, int64_t K, int32_t bits, int32_t block_size,
                    int32_t scale_dtype, int32_t out_dtype, void* stream);

/* Name of the kernel the dispatcher picks for a MatMulNBits call of this
 * geometry ("gemv_q4_mfma", "gemm_q4_mfma", "generic", ...), without touching
 * the device. Returns a static string; NULL with XRMM_EINVAL set on a bad
 * geometry. */
const char* xrmm_select_kernel(int32_t op, int64_t M, int64_t K, int64_t N, int32_t bits,
                               int32_t block_size, int32_t dtype, int32_t zp_dtype);

/* ---------------------------------------------------------------------------
 * Request-level lifecycle: the C form of xrgpu::operators::extended
 * (runtime/include/xrgpu/extended_operators.h:8-61, types
 * runtime/include/xrgpu/operators.h:9-28). Tensors carry HOST bytes here, as
 * the reference's owned Tensor does; prepare() uploads them once, run()
 * launches and waits (with the options' timeout), read_outputs() copies the
 * results back. Operation ids are "com.microsoft.MatMulNBits",
 * "com.microsoft.MatMulNBitsQkv" and "com.microsoft.MatMulNBitsMlp"; input and
 * output names are the contract's port names (aT, bT, scalesT, ...).
 * ------------------------------------------------------------------------- */

#define XRMM_MAX_RANK 16
#define XRMM_NAME_MAX 32

/* operators.h:16-23 Tensor. `data` is little-endian contiguous row-major
 * storage of `nbytes` bytes (NULL for requested outputs). */
typedef struct xrmm_tensor {
  const char* name;
  int32_t dtype;         /* logical dtype */
  int32_t storage_dtype; /* XRMM_UNSPECIFIED = same as dtype */
  int32_t rank;
  int64_t shape[XRMM_MAX_RANK];
  const void* data;
  uint64_t nbytes;
} xrmm_tensor;

/* One entry of extended_operators.h:8-17 Attributes (scalar kinds only). */
enum { XRMM_ATTR_INT = 0, XRMM_ATTR_FLOAT = 1, XRMM_ATTR_STRING = 2 };
typedef struct xrmm_attr {
  const char* key;
  int32_t kind;
  int64_t i;
  double f;
  const char* s;
} xrmm_attr;

/* extended_operators.h:22-28 Request; `args` override `attrs` by key. */
typedef struct xrmm_request {
  const char* operation;
  const xrmm_tensor* inputs;
  int32_t n_inputs;
  const xrmm_attr* attrs;
  int32_t n_attrs;
  const xrmm_attr* args;
  int32_t n_args;
  const xrmm_tensor* requested_outputs;
  int32_t n_requested_outputs;
} xrmm_request;

/* operators.h:24-28 Options (defaults: no profiling, 15 s, 256 MiB). */
typedef struct xrmm_options {
  int32_t profiling;
  uint64_t timeout_ns;
  uint64_t memory_limit_bytes;
} xrmm_options;

/* A planned output: name, dtypes, shape and storage byte count. */
typedef struct xrmm_tensor_desc {
  char name[XRMM_NAME_MAX];
  int32_t dtype;
  int32_t storage_dtype;
  int32_t rank;
  int64_t shape[XRMM_MAX_RANK];
  uint64_t nbytes;
} xrmm_tensor_desc;

typedef struct xrmm_op xrmm_op;

/* Fill `o` with the reference defaults (operators.h:24-28). */
void xrmm_default_options(xrmm_options* o);

/* extended::plan (kernels/_shared/extended/planner.cpp:67, complex branch
 * complex_plan.cpp:117-120, contract rows contract_data.h:722-751): contract
 * validation, attribute defaults, output shapes. Metadata only, no device
 * work. Writes up to `capacity` descriptors and the count to *n_outputs. */
int xrmm_plan(const xrmm_request* request, xrmm_tensor_desc* outputs, int32_t capacity,
              int32_t* n_outputs);

/* Operator::prepare (kernels/_shared/extended/vulkan.cpp:119): plan, check the
 * input byte counts and the memory limit, upload the inputs to the current
 * HIP device and create the operator's stream. */
int xrmm_prepare(const xrmm_request* request, const xrmm_options* options, xrmm_op** op);

/* Operator::run (vulkan.cpp:115,120): launch and wait up to timeout_ns. A
 * failure or time-out poisons the operator: later calls fail until close. */
int xrmm_run(xrmm_op* op);

/* Planned outputs of a prepared operator (same descriptors as xrmm_plan). */
int xrmm_output_descs(const xrmm_op* op, xrmm_tensor_desc* outputs, int32_t capacity,
                      int32_t* n_outputs);

/* Operator::read_outputs (vulkan.cpp:121): copy output i into dst[i], which
 * holds dst_bytes[i] bytes (exactly the descriptor's nbytes), converting to
 * the requested storage dtype. */
int xrmm_read_outputs(xrmm_op* op, void* const* dst, const uint64_t* dst_bytes, int32_t n);

/* Operator::info (vulkan.cpp:123): JSON with backend, device, operation,
 * closed, executed, execution_ms, gpu_ms, dispatch_count, persistent_bytes,
 * kernel. The string stays valid until the next xrmm_info or xrmm_destroy. */
const char* xrmm_info(xrmm_op* op);

/* Operator::close (vulkan.cpp:122): wait for the stream and release device
 * memory; the handle stays valid for xrmm_info until xrmm_destroy. */
int xrmm_close(xrmm_op* op);

/* Close (if open) and free the handle (the reference's destructor). */
void xrmm_destroy(xrmm_op* op);

/* ---------------------------------------------------------------------------
 * com.microsoft.QMoE, opcode 1030 (zero-copy, device pointers).
 * Replaces the serial moe path of
 * kernels/_shared/extended/shaders/complex_kernel.glsl:158-160 as planned by
 * kernels/_shared/extended/complex_plan.cpp:121-128 (inputs
 * inputT,routerT,fc1T,fc1ScalesT,fc2T,fc2ScalesT; output outputT = inputT's
 * shape). float32 input [T,H] and router [T,E]; fc1 [E,F1,H*bits/8] and fc2
 * [E,H,I*bits/8] u8, codes low-first, zero point 2^(bits-1); float32 scales
 * [E,rows] (block_size 0) or [E,rows,cols/block_size]. `activation` is
 * XRMM_ACT_RELU (swiglu_fusion 0) or XRMM_ACT_SWIGLU (swiglu_fusion 1: FC1
 * rows 2j / 2j+1 are gate / linear, I = F1/2). `workspace` is device memory of
 * at least xrmm_qmoe_workspace_bytes(T, k, H, I) bytes (routing table, the
 * activated FC1 outputs, per-slot FC2 partials and their arrival counters or
 * per-expert pair lists); calls that share a workspace must not overlap.
 * With 4- or 8-bit codes, row scales or blocks of 32 or more codes, H and I
 * multiples of 64, at most 4096 experts and at least 32 (token, slot) pairs,
 * the pairs are grouped by expert and each expert's FC1 and FC2 run as one
 * MFMA GEMM over its pairs ("qmoe_grouped"); other geometries run one pass
 * per pair ("qmoe_rows") or the scalar path. */
int64_t xrmm_qmoe_workspace_bytes(int64_t tokens, int32_t k, int64_t hidden, int64_t inter);
int xrmm_qmoe(const void* input, const void* router, const void* fc1, const void* fc1_scales, const void* fc2,
              const void* fc2_scales, void* output, void* workspace, int64_t workspace_bytes, int64_t tokens,
              int64_t hidden, int64_t experts, int64_t fc1_rows, int32_t k, int32_t bits, int32_t block_size,
              int32_t activation, int32_t swiglu_fusion, float alpha, float beta, float swiglu_limit,
              int32_t has_limit, void* stream);

/* Name of the kernel family xrmm_qmoe dispatches a geometry to
 * ("qmoe_grouped", "qmoe_rows" or "qmoe_scalar"), NULL for an invalid
 * geometry. No device work. */
const char* xrmm_qmoe_kernel(int64_t tokens, int64_t hidden, int64_t experts, int64_t fc1_rows, int32_t k, int32_t bits,
                             int32_t block_size, int32_t activation, int32_t swiglu_fusion);

/* ---------------------------------------------------------------------------
 * com.microsoft.GatherBlockQuantized, opcode 1031 (gatherQuant,
 * kernels/_shared/extended/shaders/complex_kernel.glsl:85; planner
 * complex_plan.cpp:129). data [rows, packed_cols] uint8 (codes low-first),
 * indices [n_indices] (XRMM_I32 / XRMM_U32 read as int32, or XRMM_I64
 * saturated to int32, as controlIndex does), float32 scales [rows, blocks]
 * with blocks = ceil(width / block_size), width = packed_cols * 8 / bits,
 * optional packed zero points [rows, ceil(blocks * bits / 8)] (NULL: the
 * midpoint 2^(bits-1)); output float32 [n_indices, width]. bits 4 or 8,
 * block_size a power of two >= 16. An index outside [0, rows) leaves its
 * output row zero and, when `status` (a device uint32, caller-zeroed) is not
 * NULL, raises it to 55 with an atomic max: the code the reference's run
 * fails with ("GPU operator contract validation failed: code 55",
 * vulkan.cpp:115). Enqueues on `stream` and returns. */
int xrmm_gather_block_quantized(const void* data, const void* indices, int32_t indices_dtype, const void* scales,
                                const void* zero_points, void* output, void* status, int64_t rows,
                                int64_t packed_cols, int64_t n_indices, int32_t bits, int32_t block_size,
                                void* stream);

/* com.microsoft.MatMulBnb4, opcode 1026 (bnbWeight complex_kernel.glsl:82, the
 * 1026 branch of packedMatmul :83; planner complex_plan.cpp:117-120).
 * A [M, K] and absmax [ceil(N*K / block_size)] in `dtype` (XRMM_F32 or
 * XRMM_F16), B the flat [N, K] (trans_b != 0, the default) or [K, N] weight
 * as ceil(N*K / 2) bytes, two codes per byte with the even flat index in the
 * high nibble; quant_type 1 = NF4, 0 = FP4. Y [M, N] in `dtype`. */
int xrmm_matmul_bnb4(const void* A, const void* B, const void* absmax, void* Y, int64_t M, int64_t K, int64_t N,
                     int32_t block_size, int32_t quant_type, int32_t trans_b, int32_t dtype, void* stream);

/* Kernel family xrmm_matmul_bnb4 picks ("bnb4_gemv" or "bnb4_scalar"), NULL
 * for an invalid geometry. No device work. */
const char* xrmm_matmul_bnb4_kernel(int64_t M, int64_t K, int64_t N, int32_t block_size, int32_t quant_type,
                                    int32_t trans_b, int32_t dtype);

/* Opt-in int8 activations for MatMulNBits: the upstream operator's
 * accuracy_level 4, NOT the reference's float32 arithmetic (xrGPU computes in
 * float32 at every level, complex_kernel.glsl:83). Rows of A are quantized per
 * block of 128 (scale = max|a| / 127, codes rint(a / scale)), the 4-bit
 * weights enter as signed bytes (code - zero point) and chunk sums are exact
 * int32 dot products scaled in float32. bits 4, power-of-two block_size >= 32
 * dividing K, K a multiple of 128 and at most 16384, zero points absent or packed uint8,
 * 16-byte aligned A, B and workspace (>= xrmm_matmul_nbits_int8a_workspace_bytes
 * bytes). Same argument meaning as xrmm_matmul_nbits otherwise. */
int64_t xrmm_matmul_nbits_int8a_workspace_bytes(int64_t M, int64_t K);
int xrmm_matmul_nbits_int8a(const void* A, const void* B, const void* scales, const void* zero_points,
                            int32_t zp_dtype, const void* bias, void* Y, void* workspace, int64_t workspace_bytes,
                            int64_t M, int64_t K, int64_t N, int32_t bits, int32_t block_size, int32_t dtype,
                            void* stream);

/* Allocation-free variant of xrmm_matmul_nbits_int8a. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as xrmm_matmul_nbits_int8a without the workspace:
 * the activation codes and scales go to a static device scratch of 2 MiB per
 * GPU (held until the process ends), so calls with
 * xrmm_matmul_nbits_int8a_workspace_bytes(M, K) > 2 MiB fail with XRMM_EINVAL
 * (e.g. M = 64 at K = 16384 fits). The call allocates nothing (the scratch's
 * address is looked up once per device). Every call on a GPU shares that GPU's
 * scratch: calls that overlap on one GPU (different streams, or host threads)
 * race and must be serialised by the caller. */
int xrmm_matmul_nbits_int8a_noalloc(const void* A, const void* B, const void* scales, const void* zero_points,
                                    int32_t zp_dtype, const void* bias, void* Y, int64_t M, int64_t K, int64_t N,
                                    int32_t bits, int32_t block_size, int32_t dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Measurement (no counterpart in the reference, which publishes no throughput
 * for this path): read `bytes` (a multiple of 16) at 16-byte aligned `src`
 * once with 16-byte non-temporal loads, `loads_per_lane` (1, 2, 4 or 8) per
 * lane issued back to back, and write nothing to the 4-byte `sink` in
 * practice. The plain read rate of a decode GEMV's bytes, which its time is
 * compared with. */
int xrmm_stream_read(const void* src, uint64_t bytes, void* sink, int32_t loads_per_lane, void* stream);

/* Measurement, as above, with the cache policy and grid chosen: `nontemporal`
 * 1 reads with non-temporal loads, 0 with the default policy; `workgroups` 0
 * launches the one-shot grid (every lane issues its loads once and retires),
 * a positive count launches that many 256-lane workgroups that walk the
 * buffer in strides of the whole grid (a persistent read). */
int xrmm_stream_read_ex(const void* src, uint64_t bytes, void* sink, int32_t loads_per_lane, int32_t nontemporal,
                        int32_t workgroups, void* stream);

/* Measurement (no counterpart in the reference): the sustained rate of
 * back-to-back v_mfma_f32_32x32x16_f16 on the caller's binary16 operands
 * (`operands`: xrmm_mfma_peak_operand_bytes() bytes, 16-byte aligned; random
 * values give a real GEMM's switching activity, hence its clock). Launches
 * `workgroups` workgroups of `waves` (1..4) waves, each wave issuing
 * 16 * `iters` MFMAs over `accumulators` (4 or 8) independent accumulators
 * (xrmm_mfma_peak_flops(workgroups, waves, iters) flops in total). Lane 0 of
 * global wave w writes four uint64 words to clocks[4w..4w+3]: its loop's
 * shader-clock cycles (s_memtime), the constant-rate counter (s_memrealtime)
 * at the loop's start and at its end, and its workgroup index. `sink` (4
 * bytes) is written only in the practically impossible case that the
 * accumulators sum to a fixed constant. */
int64_t xrmm_mfma_peak_operand_bytes(void);
int64_t xrmm_mfma_peak_flops(int32_t workgroups, int32_t waves, int32_t iters);
int xrmm_mfma_peak(const void* operands, void* sink, void* clocks, int32_t workgroups, int32_t waves,
                   int32_t accumulators, int32_t iters, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* XRMM_H */
