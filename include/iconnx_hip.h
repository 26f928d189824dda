/*
 * iconnx_hip — MI355X (gfx950) kernels for iconnx's dynamically-quantized linear path.
 *
 * C ABI: plain device pointers and sizes, no framework types.  Every compute entry point
 * enqueues on `stream` and returns an icx_status; nothing synchronises the host unless
 * stated.  Device pointers are caller-owned.  Scalars that live on the device in the
 * reference (DQL's y_scale / y_zero_point outputs, MatMulInteger zero points) are device
 * pointers here too, so a DQL -> MatMulInteger chain never round-trips through the host.
 *
 * Each declaration names the reference interface (path:line in ryanoneill/iconnx) whose
 * role it takes over.  The reference's Rust wrappers would bind these through an
 * `extern "C"` block declaring the same signatures.
 */
#ifndef ICONNX_HIP_H
#define ICONNX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* icx_stream_t; /* == hipStream_t */

/* ---- status / errors (mirrors CudaError::Kernel(String), src/cuda/context.rs) ------- */
typedef enum {
    ICX_OK = 0,
    ICX_ERR_INVALID_ARG = 1, /* null pointer, zero-sized where not allowed */
    ICX_ERR_SHAPE = 2,       /* shape contract violated (K mismatch, zp length, ...) */
    ICX_ERR_DTYPE = 3,       /* dtype contract violated (non-f32 DQL input, ...) */
    ICX_ERR_WORKSPACE = 4,   /* workspace missing or smaller than the *_workspace_size */
    ICX_ERR_HIP = 5,         /* a HIP runtime call failed */
    ICX_ERR_UNSUPPORTED = 6, /* outside what this build implements */
    ICX_ERR_KERNEL = 7,      /* a kernel reported a failure on the device (icx_graph_status) */
} icx_status;

/* ICX_I64: Reshape shapes (graph initializers, read on the host) and Gather indices / data.
 * ICX_BOOL: one byte per element, 0 or 1 (ONNX BOOL; Equal's output, Where's condition). */
typedef enum { ICX_I8 = 0, ICX_U8 = 1, ICX_I32 = 2, ICX_F32 = 3, ICX_I64 = 4, ICX_BOOL = 5 } icx_dtype;

const char* icx_status_str(int status);
/* Message of the last failing call on this host thread ("" if none). */
const char* icx_last_error(void);
/* Library / build identification, e.g. "iconnx_hip gfx950 ...". */
const char* icx_version(void);

/* ---- streams, memory, transfers --------------------------------------------------------
 * What garboard and IconnxCudaContext / GpuMemoryPool give the reference's wrappers.
 * icx_stream_create: the context's one stream (src/cuda/context.rs:28-31), default priority.
 * icx_stream_synchronize: IconnxCudaContext::sync (context.rs:226-232). */
int icx_stream_create(icx_stream_t* out);
int icx_stream_destroy(icx_stream_t stream);
int icx_stream_synchronize(icx_stream_t stream);

/* GpuMemoryPool (src/cuda/memory_pool.rs:47-545) on hipMalloc.  icx_pool_alloc is get_f32 /
 * get_u8 / get_i32 / ... (:104-400): a buffer of at least `bytes` bytes of a power-of-two size
 * class (>= 256 B), from the pool or fresh on a miss; NOT zero-filled (the reference clears
 * reused slices, :120; every kernel here writes its whole output).  icx_pool_free is
 * return_tensor (:482): at most eight free buffers are kept per class, as max_per_bucket
 * (:94), and a buffer beyond that is freed; a pointer this pool did not hand out is
 * ICX_ERR_INVALID_ARG.  Buffers are reused in stream order: return one once the last work
 * reading it is enqueued on the stream that will use it next.  icx_pool_stats is stats()
 * (:526): hits, misses (hipMalloc calls) and bytes held.  icx_pool_destroy frees every buffer,
 * handed out or not.  A pool is used from one host thread at a time (the reference's
 * executor is !Sync). */
typedef struct icx_pool icx_pool;
icx_pool* icx_pool_create(void);
void icx_pool_destroy(icx_pool* pool);
int icx_pool_alloc(icx_pool* pool, size_t bytes, void** out);
int icx_pool_free(icx_pool* pool, void* ptr);
int icx_pool_stats(icx_pool* pool, int64_t* hits, int64_t* misses, int64_t* bytes_held);

/* IconnxCudaContext::htod / dtoh (context.rs:160-223) as stream-ordered copies: both return
 * once enqueued (the reference's dtoh blocks the host).  With pinned host memory from
 * icx_host_alloc the copy runs asynchronously; the destination of a D2H copy is valid after
 * icx_stream_synchronize. */
int icx_host_alloc(size_t bytes, void** out);
int icx_host_free(void* ptr);
int icx_memcpy_h2d_async(icx_stream_t stream, void* dst, const void* src, size_t bytes);
int icx_memcpy_d2h_async(icx_stream_t stream, void* dst, const void* src, size_t bytes);

/* ---- DynamicQuantizeLinear ------------------------------------------------------------
 * Replaces gpu_dynamic_quantize_linear (src/cuda/ops/quantize.rs:296-377), which copies x to
 * the host; semantics of DynamicQuantizeLinear::forward
 * (src/operators/dynamic_quantize_linear.rs:32-112): min/max over x with 0 included and NaN
 * skipped, scale = (max-min)/255 and the zero point in f64, y = clamp(rne(x/scale) + zp)
 * with the division in f64; min == max gives y = 0, scale 0, zp 0.
 * Outputs y[n] (u8), *y_scale (f32, device), *y_zp (u8, device).
 * opt_rowsum (nullable): when given, rowsum[r] = sum of y over row r of an [n/row_len,
 * row_len] view (u8 values summed as int32) — the row term a downstream MatMulInteger
 * needs for a non-zero b zero point.  row_len must divide n.
 * ws: device workspace of icx_dql_workspace_size(n) bytes (no initialisation needed). */
size_t icx_dql_workspace_size(size_t n);
int icx_dynamic_quantize_linear(icx_stream_t stream, const float* x, size_t n, uint8_t* y,
                                float* y_scale, uint8_t* y_zp, int32_t* opt_rowsum,
                                size_t row_len, void* ws, size_t ws_bytes);

/* The same op as one launch (no counterpart in the reference, whose op runs as its two
 * kernels; for callers that keep one buffer per stream): every block keeps its slice of x in
 * registers and the blocks trade their (min, max) through `sync`, a buffer of
 * icx_exchange_buffer_size() bytes that the caller zeroes once before its first use and
 * keeps for later calls (it carries a launch number from call to call; calls sharing a
 * buffer must not overlap).  Same outputs, bit for bit, as icx_dynamic_quantize_linear
 * without row sums.  Up to 4 Mi elements (1024 resident blocks of 256 lanes with 4 float4
 * each), x 16-byte and y 4-byte aligned: otherwise ICX_ERR_UNSUPPORTED with nothing
 * launched.  All blocks must run at once: if other work keeps some from being scheduled,
 * the waiting blocks give up after a bounded time, write y as 0 and the scale as NaN, and
 * the next icx_exchange_status on the buffer returns ICX_ERR_KERNEL. */
size_t icx_exchange_buffer_size(void);
int icx_dynamic_quantize_linear_exchange(icx_stream_t stream, const float* x, size_t n, uint8_t* y,
                                         float* y_scale, uint8_t* y_zp, void* sync);
/* Synchronise the stream, then report (ICX_ERR_KERNEL) and clear the failures recorded in
 * an exchange buffer since the last check. */
int icx_exchange_status(icx_stream_t stream, void* sync);

/* ---- weight packing (once per weight; part of initializer upload in the reference,
 * src/ir/lowering.rs:292-297) -----------------------------------------------------------
 * B [K,N] row-major (i8 or u8) -> packed [N,K] i8 (u8 shifted by -128) + colsum[N] of the
 * packed values.  packed needs icx_packed_weight_bytes(K,N) bytes. */
size_t icx_packed_weight_bytes(size_t K, size_t N);
int icx_pack_weight(icx_stream_t stream, const void* B, int b_dtype, size_t K, size_t N,
                    int8_t* packed, int32_t* colsum);

/* ---- MatMulInteger -------------------------------------------------------------------
 * Replaces gpu_matmul_integer (src/cuda/ops/quantize.rs:398-615) and its naive kernels
 * (src/cuda/ops/quantize_kernels.rs:116-194); semantics of MatMulInteger::forward
 * (src/operators/matmul_integer.rs:52-267): C[m,n] = sum_k (A[m,k]-a_zp)(B[k,n]-b_zp)
 * in int32 (wrapping).  A [M,K] row-major i8/u8.  B either row-major [K,N]
 * (b_packed = 0; packed into the workspace on every call) or the output of
 * icx_pack_weight (b_packed = 1, colsum required).  a_zp: device scalar in A's dtype or
 * NULL (0).  b_zp: device array in B's dtype of length b_zp_len (1 = per-tensor, as in the
 * reference; N = per-column, the ONNX form the reference rejects) or NULL.
 * a_rowsum (nullable): sum of raw A over each row (e.g. from icx_dynamic_quantize_linear);
 * computed into the workspace when needed and absent.
 * ws: icx_matmul_integer_workspace_size(...) bytes. */
size_t icx_matmul_integer_workspace_size(size_t M, size_t K, size_t N, int b_packed);
int icx_matmul_integer(icx_stream_t stream, const void* A, int a_dtype, const void* B,
                       int b_dtype, int b_packed, const int32_t* b_colsum, size_t M,
                       size_t K, size_t N, const void* a_zp, const void* b_zp,
                       size_t b_zp_len, const int32_t* a_rowsum, int32_t* C, void* ws,
                       size_t ws_bytes);

/* No counterpart in the reference: icx_matmul_integer for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * calls no allocator: the workspace icx_matmul_integer would take lives in a static device
 * array of icx_matmul_integer_noalloc_max_bytes() bytes (32 MiB) per GPU, held until the
 * process ends.  Arguments and results as icx_matmul_integer; a shape whose workspace
 * (icx_matmul_integer_workspace_size) exceeds that size is ICX_ERR_WORKSPACE, before any
 * GPU work.  Calls that overlap on one GPU (two streams or host threads) share the array
 * and race: order them. */
size_t icx_matmul_integer_noalloc_max_bytes(void);
int icx_matmul_integer_noalloc(icx_stream_t stream, const void* A, int a_dtype, const void* B,
                               int b_dtype, int b_packed, const int32_t* b_colsum, size_t M,
                               size_t K, size_t N, const void* a_zp, const void* b_zp,
                               size_t b_zp_len, const int32_t* a_rowsum, int32_t* C);

/* ---- elementwise epilogue / fused chain -----------------------------------------------
 * An ordered list of f32 binary ops applied to a running value v, each rounding once,
 * exactly like separate ONNX Mul/Add/Sub/Div nodes (src/operators/{mul,add,div}.rs):
 *   v = op(v, operand)   or, with operand_is_lhs, v = op(operand, v).
 * An operand broadcasts over the [rows, cols] output: a device scalar, a [cols] vector, a
 * [rows] vector or a full [rows, cols] tensor.  It may be the product of two such factors
 * (p1 != NULL), rounded once — the Mul(x_scale, w_scale) node feeding the dequant Mul.
 * Replaces the reference's MulAdd / AddMul / SubMul / DivMul fused kernels
 * (src/cuda/kernels/fused/mod.rs:290-378, wrappers.rs:495-683) and the unfused
 * Mul/Add/Div broadcast path (src/cuda/executor/elementwise.rs:54-200), with [cols]
 * broadcast allowed everywhere (the reference DivMul requires equal shapes). */
enum { ICX_OP_ADD = 0, ICX_OP_SUB = 1, ICX_OP_MUL = 2, ICX_OP_DIV = 3 };
/* Operand-free steps (p0 may be NULL; kinds ignored), for the erf-GELU subgraph
 * Mul(x, Add(Erf(Div(x, c0)), c1)) [* c2] (src/operators/erf.rs:21-31):
 *   ICX_OP_ERF        v = erf(v) — the reference's Abramowitz-Stegun 7.1.26 in f32, with a
 *                     Newton-refined hardware reciprocal and the hardware exp2 (within 2e-7
 *                     of the formula evaluated with correctly rounded ops);
 *   ICX_OP_SAVE       s = v (v unchanged);
 *   ICX_OP_MUL_SAVED  v = s * v (one rounding; operand_is_lhs ignored, products commute).
 * A Div (operand on the right) whose next step is ICX_OP_ERF is, in chains whose operands
 * are all scalars or [cols] vectors, evaluated as v * RN(1 / operand): at most one ulp from
 * the quotient, which moves the erf result by < 4e-8 (its only reader; Erf is compared
 * within tolerance anyway).  Every other step rounds exactly as the reference's node. */
enum { ICX_OP_ERF = 4, ICX_OP_SAVE = 5, ICX_OP_MUL_SAVED = 6 };
enum { ICX_BCAST_SCALAR = 0, ICX_BCAST_COL = 1, ICX_BCAST_ROW = 2, ICX_BCAST_FULL = 3 };
#define ICX_MAX_CHAIN 8

typedef struct {
    int32_t op;             /* ICX_OP_* */
    int32_t operand_is_lhs; /* 1: v = operand op v */
    int32_t kind0, kind1;   /* ICX_BCAST_* of p0 / p1 */
    const float* p0;        /* device pointer */
    const float* p1;        /* optional second factor (device) or NULL */
} icx_chain_op;

typedef struct {
    int32_t n_ops; /* 0..ICX_MAX_CHAIN */
    int32_t reserved;
    icx_chain_op ops[ICX_MAX_CHAIN];
} icx_chain;

/* Y[rows,cols] = chain(X).  X and Y may alias. */
int icx_fused_chain_f32(icx_stream_t stream, const float* X, size_t rows, size_t cols,
                        const icx_chain* chain, float* Y);

/* Quantized linear with the epilogue fused into the GEMM store:
 * Y = chain(Cast<float>(MatMulInteger(A, B, a_zp, b_zp))).  Arguments as for
 * icx_matmul_integer; chain may be NULL (plain Cast). */
int icx_qlinear_f32(icx_stream_t stream, const void* A, int a_dtype, const void* B,
                    int b_dtype, int b_packed, const int32_t* b_colsum, size_t M, size_t K,
                    size_t N, const void* a_zp, const void* b_zp, size_t b_zp_len,
                    const int32_t* a_rowsum, const icx_chain* chain, float* Y, void* ws,
                    size_t ws_bytes);

/* DynamicQuantizeLinear of x [M, K] and the quantized linear that reads its output, as ONE
 * launch (no counterpart in the reference, which runs the DQL's host loop and then the
 * linear's nodes): y, y_scale, y_zp are icx_dynamic_quantize_linear(x)'s outputs and Y is
 * icx_qlinear_f32(A = y, a_zp = y_zp, packed Int8 B, colsum, no b zero point, chain)'s, bit
 * for bit; the chain reads the activation scale as the scalar y_scale (e.g. its first op
 * Mul(y_scale * w_scale)).  The GEMM's blocks compute the range of their slices of x, trade
 * it through `sync` (an icx_exchange_buffer_size() buffer, as for
 * icx_dynamic_quantize_linear_exchange: zeroed once, kept, calls sharing it must not overlap),
 * quantize their slices into y and wait only for the slices of their own row panel.
 * K % 128 == 0 and N % 96 == 0 (256x192 tiles where each block's share of its 256-row panel
 * fits its registers, 4 * 4 * 768 floats, else 64x96 tiles, 4 * 4 * 384), column-only chain
 * (the erf-GELU on 256x192 tiles only), x / y / B 16-byte aligned, every block resident at
 * once (at most 1024): otherwise
 * ICX_ERR_UNSUPPORTED with nothing launched (call the two entry points instead).  A wait
 * that runs out (blocks kept from running by other work) is reported by icx_exchange_status
 * as ICX_ERR_KERNEL, with y_scale NaN. */
int icx_dql_qlinear_f32(icx_stream_t stream, const float* x, size_t M, size_t K, uint8_t* y,
                        float* y_scale, uint8_t* y_zp, const void* B, int b_dtype,
                        const int32_t* b_colsum, size_t N, const icx_chain* chain, float* Y,
                        void* sync);

/* Cast INT32 -> FLOAT (src/operators/cast.rs:46-49; GPU src/cuda/ops/cast.rs:134-148). */
int icx_cast_i32_f32(icx_stream_t stream, const int32_t* x, size_t n, float* y);

/* ---- DequantizeLinear ---------------------------------------------------------------
 * Replaces gpu_dequantize_linear (src/cuda/ops/quantize.rs:24-267); semantics of the CPU
 * DequantizeLinear::forward (src/operators/dequantize_linear.rs:32-180):
 * y = (x as f32 - zp as f32) * scale with the per-axis index (i / inner) % axis_size.
 * x: i8/u8/i32; zp: same dtype, length axis_size, or NULL. */
int icx_dequantize_linear_f32(icx_stream_t stream, const void* x, int x_dtype,
                              const float* scale, const void* zp, size_t n,
                              size_t axis_size, size_t inner, float* y);

/* ---- Gather --------------------------------------------------------------------------
 * Replaces gpu_gather_from_gpu / gpu_gather (src/cuda/ops/layout/mod.rs:689-1020) and its
 * kernels (gather_kernel / gather_i64_kernel, and gather_u8_kernel,
 * src/cuda/ops/quantize_kernels.rs:203-224, which DistilBERT-INT8's UINT8 word-embedding table
 * goes through); ONNX Gather semantics of src/operators/gather.rs:21-205 on any element type:
 * data viewed as [outer, axis_len, inner] elements of elem_bytes bytes (outer = product of the
 * dims before `axis`, inner = after), out [outer, n_idx, inner] with out[o, i, :] =
 * data[o, k, :], k = indices[i] (+ axis_len when negative), clamped into [0, axis_len - 1]
 * as the reference's kernels do.  indices: device Int64 (ICX_I64) or Int32 (ICX_I32). */
int icx_gather(icx_stream_t stream, const void* data, size_t elem_bytes, size_t outer,
               size_t axis_len, size_t inner, const void* indices, int idx_dtype, size_t n_idx,
               void* out);

/* ---- encoder ops (fp32) --------------------------------------------------------------
 * The fp32 ops a DistilBERT-shaped encoder needs around its quantized linears.  Parity: the
 * f32 reductions follow the reference's CPU order where it is defined by its own code
 * (LayerNormalization, Softmax: ndarray's eight-way unrolled sum); exp and the MatMul
 * summation order are the device's, so those outputs match the reference within f32
 * rounding tolerance rather than bit for bit. */

/* LayerNormalization over the last axis (src/operators/layer_normalization.rs:25-80) of
 * x [rows, cols], or of (x + residual) when residual is not NULL (the Add feeding the norm,
 * one f32 rounding).  scale, bias: [cols], or NULL for none (x * 1 and x + (-0.0), which
 * change no bit: the node-by-node form ReduceMean -> Sub -> Pow -> ReduceMean -> Add ->
 * Sqrt -> Div without its Mul / Add tail). */
int icx_layer_norm_f32(icx_stream_t stream, const float* x, const float* residual, size_t rows,
                       size_t cols, const float* scale, const float* bias, float eps, float* y);

/* Softmax over the last axis (src/operators/softmax.rs:25-40).  x and y must not alias. */
int icx_softmax_f32(icx_stream_t stream, const float* x, size_t rows, size_t cols, float* y);

/* ReduceMean (src/operators/reduce_mean.rs:19-105; GPU gpu_reduce_mean_axis,
 * src/cuda/reduction.rs:623-700, dispatched by src/cuda/executor/reduction.rs:88-104) of x
 * viewed as [outer, axis_len, inner] over its middle axis: y [outer, inner] = sum / axis_len
 * (the length converted to f32, one division).  The sum follows ndarray 0.16's order:
 * sequential == 0 — the contiguous last axis (inner must be 1), or every element of x as one
 * lane (outer = inner = 1) — unrolled_fold's eight partial sums; sequential != 0 — any other
 * axis — 0 + x[.., 0, ..] + x[.., 1, ..] + ... in order.  axis_len == 0 is ICX_ERR_SHAPE (the
 * reference's mean_axis returns None and it panics). */
int icx_reduce_mean_f32(icx_stream_t stream, const float* x, size_t outer, size_t axis_len,
                        size_t inner, int sequential, float* y);

/* Pow (src/operators/pow.rs:18-45; GPU: the "Pow" arm of src/cuda/executor/elementwise.rs:
 * 194-230): y [rows, cols] = x ^ e, the exponent broadcast over x as e_kind (ICX_BCAST_*:
 * scalar, [cols], [rows] or full).  An exponent of exactly 2 gives the correctly rounded
 * square x * x; any other the device powf.  The reference CPU calls the C library's powf
 * (glibc 2.35 here), which is not correctly rounded: for exponent 2 it differs from x * x in
 * the last bit for ~0.07 % of inputs, so Pow matches it within one ulp, not bit for bit. */
int icx_pow_f32(icx_stream_t stream, const float* x, size_t rows, size_t cols, const float* e,
                int e_kind, float* y);

/* Sqrt (src/operators/sqrt.rs:18-30; GPU: the "Sqrt" arm of src/cuda/executor/
 * elementwise.rs:233-250): y = sqrt(x), correctly rounded like f32::sqrt. */
int icx_sqrt_f32(icx_stream_t stream, const float* x, size_t n, float* y);

/* Transpose (src/operators/transpose.rs:10-40): y = x.permuted_axes(perm), standard layout;
 * rank <= 6; elements of 1 or 4 bytes. */
int icx_transpose(icx_stream_t stream, const void* x, size_t elem_bytes, int rank,
                  const int64_t* dims, const int* perm, void* y);

/* Batched f32 MatMul (src/operators/matmul.rs:20-150): c[i] = a[i] @ b[b_broadcast ? 0 : i],
 * a [M,K], b [K,N], all row-major; batch <= 65535. */
int icx_matmul_f32(icx_stream_t stream, const float* a, const float* b, size_t batch,
                   int b_broadcast, size_t M, size_t K, size_t N, float* c);

/* Fused self-attention over [B, S, H*D] activations (row strides ld*, elements): for every
 * (b, h), out[b, s, h*D + d] = sum_c softmax_c(score[s, c]) * v[b, c, h*D + d] with
 * score[s, c] = sum_d q[b, s, h*D + d] * k[b, c, h*D + d], scaled by `scale` (division when
 * scale_div, else multiplication), applied to q before the product when scale_q, else to the
 * scores.  This is the BERT subgraph Reshape -> Transpose -> MatMul -> Div|Mul -> Softmax ->
 * MatMul -> Transpose -> Reshape the reference runs node by node
 * (src/operators/{reshape,transpose,matmul,div,softmax}.rs).  D == 64, S <= 8192 (up to 128
 * keys in one tile with the exact row max; longer sequences in 128-key chunks with a running
 * softmax, the same result within f32 rounding). */
int icx_attention_f32(icx_stream_t stream, const float* q, const float* k, const float* v,
                      size_t B, size_t S, size_t H, size_t D, size_t ldq, size_t ldk,
                      size_t ldv, size_t ldo, float scale, int scale_div, int scale_q,
                      float* out);

/* ---- graph executor ------------------------------------------------------------------
 * Mirrors GpuGraphExecutor (src/cuda/inference/mod.rs:208-659): add_input (:306),
 * add_initializer (:317), add_node (:331), a lowering step (ir::lower,
 * src/ir/lowering.rs:31-238: topological sort, fusion decision, initializer upload) and run
 * (:428) with the input-shape guard (:441-460).  Ops dispatched: DynamicQuantizeLinear,
 * MatMulInteger (2-D and 3-D x 2-D, layout.rs:1034-1095), DequantizeLinear, Cast (to
 * FLOAT / INT32 / INT64 / BOOL), Mul / Add / Sub / Div, the encoder's LayerNormalization,
 * ReduceMean, Pow, Sqrt, Softmax, Erf, Transpose, Reshape (the output aliases the input) and
 * f32 MatMul, Gather, and an export's shape / mask plumbing: Shape, Unsqueeze, Squeeze,
 * Identity, Concat, Slice, Expand, Equal, Where (integer tensors known on the host — Shape
 * results, small initializers, inputs bound from host memory — are computed on the host, as
 * the reference's get_or_fetch_i64 cache and shape-extraction folding do; the rest runs on
 * the device); anything else is an ICX_ERR_UNSUPPORTED error naming the node.
 * Fused patterns (src/cuda/inference/fusion/patterns.rs:15-109 plus one new head):
 *   QuantizedLinear  MatMulInteger -> Cast -> Mul(scale or Mul(x_scale, w_scale)) [-> Add]
 *                    [-> Mul/Add/Sub/Div with static operands]*
 *                    [-> erf-GELU: Div, Erf, Add, Mul(x, .), Mul]      => icx_qlinear_f32
 *   MulAdd / AddMul / SubMul / DivMul / ElementwiseChain / Gelu — chains of elementwise ops
 *                    with static operands (scalar, [last dim], same shape) => icx_fused_chain_f32
 *   Attention        Reshape -> Transpose -> MatMul -> Div|Mul -> [Where(padding mask,
 *                    fill, .)] -> Softmax -> MatMul -> Transpose -> Reshape of a
 *                    self-attention (reshape targets may be computed at run time, the key
 *                    transposed twice) => the attention kernel, or the nodes one by one when
 *                    the shapes or the mask fall outside it
 *   AddLayerNorm     LayerNormalization(Add(a, b)) => icx_layer_norm_f32 with a residual
 *   DecomposedLayerNorm  the same written node by node (ReduceMean / Sub / Pow / Sqrt / Div)
 *   GatherDequantize DequantizeLinear(Gather(UInt8 / Int8 table, indices)), per-tensor scale
 * Attribute values are int64 (axis, to); names of absent optional inputs are "". */
typedef struct icx_graph icx_graph;

icx_graph* icx_graph_create(void);
void icx_graph_destroy(icx_graph* g);
/* dims: rank entries; -1 marks a dynamic dimension (shape[i] == None in the reference). */
int icx_graph_add_input(icx_graph* g, const char* name, int rank, const int64_t* dims);
/* Host data is copied (uploaded at compile).  dtype: ICX_I8 / ICX_U8 / ICX_I32 / ICX_F32 /
 * ICX_I64 / ICX_BOOL. */
int icx_graph_add_initializer(icx_graph* g, const char* name, int dtype, int rank,
                              const int64_t* dims, const void* host_data);
int icx_graph_add_node(icx_graph* g, const char* name, const char* op_type, int n_in,
                       const char* const* inputs, int n_out, const char* const* outputs,
                       int n_attr, const char* const* attr_names, const int64_t* attr_values);
/* Non-integer attributes of an added node: a float (LayerNormalization epsilon) or a list
 * of ints (Transpose perm, Unsqueeze / Squeeze / ReduceMean axes). */
int icx_graph_set_node_attr_float(icx_graph* g, const char* node, const char* attr, double value);
int icx_graph_set_node_attr_ints(icx_graph* g, const char* node, const char* attr, int count,
                                 const int64_t* values);
int icx_graph_add_output(icx_graph* g, const char* name);
/* A planner option (no counterpart in the reference, whose nodes always run one by one):
 *   "quantized_outputs" 1 (default) / 0 — whether a head whose output only a
 *   DynamicQuantizeLinear reads (quantized linear, attention) may write that DQL's outputs
 *   itself in the same launch, and a quantized linear may run the DQL of its own input
 *   (icx_dql_qlinear_f32's kernel); 0 runs every DQL as its own launch (the results are
 *   bit-identical either way; the option isolates the fused kernels when checking that).
 *   "quantized_inputs" 1 (default) / 0 — the second part alone.
 * ICX_ERR_INVALID_ARG for an unknown name or value.  Takes effect at the next plan. */
int icx_graph_set_option(icx_graph* g, const char* name, int64_t value);
/* Host passes only (topological sort, fusion decision, zero-point folding); no GPU work.
 * Writes a text summary into buf (may be NULL): one "<node> <op> <kind> <pattern> [k=v...]"
 * line per executed op in order (kind Regular or FusedHead; a head's fused nodes follow it as
 * Skip lines), then one "rowsum <tensor>" line per DQL output whose row sums are emitted. */
int icx_graph_plan(icx_graph* g, char* buf, size_t buf_len);
/* Plan (if needed), upload initializers, pack MatMulInteger weights (colsums), on stream. */
int icx_graph_compile(icx_graph* g, icx_stream_t stream);
/* Bind an input: `data` is host memory (copied H2D on the stream) or, with on_device = 1, a
 * device pointer used in place. */
int icx_graph_set_input(icx_graph* g, const char* name, int dtype, int rank, const int64_t* dims,
                        const void* data, int on_device);
int icx_graph_run(icx_graph* g, icx_stream_t stream);
/* Device pointer / dtype / shape of an output after run (valid until the next run). */
int icx_graph_get_output(icx_graph* g, const char* name, int* dtype, int* rank, int64_t* dims,
                         const void** device_ptr);
/* One eager run with per-op timing (GpuGraphExecutor::run_with_profiling,
 * src/cuda/inference/mod.rs:649-658; Executor::run_with_profiling,
 * src/cuda/executor/variants.rs:415-515; GpuEventTimer, src/cuda/inference/gpu_event_timer.rs:
 * 61-117): a hipEvent is recorded after the input uploads and after each executed op, the
 * stream is synchronised once, and op k's gpu_us is the interval between its event and the
 * previous one.  Records go to ops[0 .. min(capacity, n) - 1] in execution order; *n_ops =
 * the number of executed ops; *upload_us (may be NULL) = the input uploads' GPU time.  Not
 * for a captured graph (the events would be recorded into it): it runs eagerly like
 * icx_graph_run, with the same outputs. */
typedef struct icx_op_profile {
    char label[48]; /* the op type, or "Fused_<pattern>" for a fused head (the reference's op_label) */
    char node[80];  /* the planned op's node name (truncated) */
    float gpu_us;   /* device time of its kernels */
    float cpu_us;   /* host time to validate and enqueue it */
} icx_op_profile;
int icx_graph_run_profiled(icx_graph* g, icx_stream_t stream, icx_op_profile* ops, int capacity,
                           int* n_ops, float* upload_us);
/* Memory pool statistics: allocations from hipMalloc, pool hits, bytes held. */
int icx_graph_pool_stats(icx_graph* g, int64_t* hipmallocs, int64_t* hits, int64_t* bytes_held);
/* Record one run into a HIP graph for repeated inference (no counterpart in the reference,
 * whose GpuGraphExecutor::run, src/cuda/inference/mod.rs:428, launches every kernel from
 * the host on each call).  Every input must be bound
 * on the device (icx_graph_set_input with on_device = 1): the graph reads those pointers in
 * place, so new data is written into the same buffers before a replay.  A warm-up run
 * executes first (sizing the pool and the workspace); the recorded run does not execute.
 * Changing a bound device pointer, shape or dtype, or adding to the graph, drops the
 * recording.  `stream` must be a created stream (the legacy default stream cannot be
 * captured).  Replays and runs of one graph must be ordered on one stream. */
int icx_graph_capture(icx_graph* g, icx_stream_t stream);
/* Launch the recorded run on `stream`; outputs as after icx_graph_run. */
int icx_graph_replay(icx_graph* g, icx_stream_t stream);
/* Synchronise `stream`, then report failures that kernels of earlier runs / replays of this
 * graph recorded on the device; the reference surfaces a failed launch as
 * CudaError::Kernel (src/cuda/executor/mod.rs:169-186).  icx_graph_run and icx_graph_replay
 * only enqueue work, so a failure that happens on the device can only be seen here.  The one
 * such failure today: a quantized linear that quantizes its own output (the 'quantout'
 * pairs of icx_graph_plan) needs every block of its launch resident at once; the launch is
 * sized from the occupancy calculator, so other work on the GPU at the same time can keep
 * blocks from being scheduled, and a block whose bounded wait for the others runs out
 * writes its part of the u8 output as 0 and the scale as NaN.  Returns ICX_ERR_KERNEL (and
 * clears the record) if that happened in any launch since the last call, else ICX_OK. */
int icx_graph_status(icx_graph* g, icx_stream_t stream);

/* ---- test hooks ------------------------------------------------------------------------
 * No counterpart in the reference.  icx_debug_qout_fault(us): with us > 0, every later
 * exchange launch of this process (quantized-output GEMM, single-launch DQL) waits for a tag
 * that no block publishes and gives up after `us` microseconds (instead of the normal
 * 20 ms), so every block takes the failure path and exits normally (for testing
 * icx_graph_status); 0 restores normal launches. */
void icx_debug_qout_fault(int us);

#ifdef __cplusplus
}
#endif
#endif /* ICONNX_HIP_H */
