// Library-internal entry points the graph executor uses (not part of the C ABI): the
// producers of a DynamicQuantizeLinear input can leave the DQL range partials of their
// output (see range_acc in icx_common.hpp), and the DQL then runs its quantize launch only.
#pragma once

#include "icx_common.hpp"

namespace icx {

// Compute units of the current device (cached per device; 256 if the query fails).
inline int num_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// icx_layer_norm_f32 leaving up to kMaxRangeParts (min, max) partials of y in `part`
// (may be null); *n_part = partials written, 0 when this shape's kernel leaves none.
// res_rows != 0: the residual has res_rows rows (dividing rows), row r of x adding residual
// row r % res_rows — a [S, cols] table broadcast over [B, S, cols].
int layer_norm_f32(hipStream_t s, const float* x, const float* residual, size_t res_rows, size_t rows, size_t cols,
                   const float* scale, const float* bias, float eps, float* y, float2* part, int* n_part);

// Longest sequence of the fused attention (up to 128 keys in one tile, longer ones in chunks
// of 128 with a running softmax); head size 64.
constexpr int kAttentionMaxSeq = 8192;

// An exported attention's padding mask, Where(mask, fill, scores) before the Softmax with a
// mask that broadcasts as [B, 1, 1, S]: key j of batch b is masked when keys[b * batch_stride
// + j] != 0 (batch_stride 0: one row for every batch); a masked score becomes `fill`.
struct AttnMask {
    const uint8_t* keys = nullptr;
    int64_t batch_stride = 0;
    float fill = 0.0f;
};

// icx_attention_f32 (mask: null, or an AttnMask) with the same partial output.
int attention_f32(hipStream_t s, const float* q, const float* k, const float* v, size_t B, size_t S,
                  size_t H, size_t D, size_t ldq, size_t ldk, size_t ldv, size_t ldo, float scale,
                  int scale_div, int scale_q, const AttnMask* mask, float* out, float2* part, int* n_part);

// The attention of icx_attention_f32 followed by a DynamicQuantizeLinear of its output, as
// one launch: y [B * S, row stride ldo] u8, y_scale, y_zp are what the DQL of the f32
// context would give, bit for bit, and the context itself is never written.  The blocks
// trade their ranges through `sync` (qlinear_dql's exchange, same contract and failure
// reporting).  ICX_ERR_UNSUPPORTED, having launched nothing, for a grid that would not be
// resident at once.
int attention_dql(hipStream_t s, const float* q, const float* k, const float* v, size_t B, size_t S,
                  size_t H, size_t D, size_t ldq, size_t ldk, size_t ldv, size_t ldo, float scale,
                  int scale_div, int scale_q, const AttnMask* mask, uint8_t* y, float* y_scale, uint8_t* y_zp,
                  unsigned* sync);

// icx_qlinear_f32 with the same partial output.
int qlinear_f32(hipStream_t s, const void* A, int a_dtype, const void* B, int b_dtype, int b_packed,
                const int32_t* b_colsum, size_t M, size_t K, size_t N, const void* a_zp, const void* b_zp,
                size_t b_zp_len, const int32_t* a_rowsum, const icx_chain* chain, float* Y, void* ws,
                size_t ws_bytes, float2* part, int* n_part);

// Sibling quantized linears over one input in one launch: B is the packed weight of the
// column-concatenated [K, N] weight, N = n_seg equal segments of a multiple of 256 columns,
// segment s (columns [s*N/n_seg, (s+1)*N/n_seg)) stored as the row-major [M, N/n_seg]
// tensor ys[s].  Column chain operands index the concatenated N.
int qlinear_f32_seg(hipStream_t s, const void* A, int a_dtype, const void* B, int b_dtype,
                    const int32_t* b_colsum, size_t M, size_t K, size_t N, const void* a_zp, const void* b_zp,
                    size_t b_zp_len, const int32_t* a_rowsum, const icx_chain* chain, float* const* ys,
                    int n_seg, void* ws, size_t ws_bytes);

// A quantized linear whose f32 output is read only by a DynamicQuantizeLinear, as one launch:
// y, y_scale, y_zp are what the DQL of icx_qlinear_f32's Y would give, bit for bit, and Y
// itself is never written.  Int8 packed weight without zero point (no row term), column-only
// chain, K % 128 == 0, N % 192 == 0, 16-byte aligned A, B and y, at most kQoutMaxBlocks
// 256x192 tiles.  `sync`: kQoutSyncBytes of device memory, zero before its first use and
// left valid by every call; calls that share it must not overlap.  Returns
// ICX_ERR_UNSUPPORTED, having launched nothing, for a shape outside the kernel or a grid
// that would not be resident at once.
constexpr int kQoutMaxBlocks = 1024;  // blocks of one quantized-output launch
// qexchange.hpp's layout: words and the launch's result, a tagged pair per block, 9 counters,
// a tagged word per block
constexpr size_t kQoutSyncBytes = 256 + 16 * (size_t)kQoutMaxBlocks + 9 * 128 + 4 * (size_t)kQoutMaxBlocks;
constexpr int kQoutErrWord = 2;  // word of that buffer counting launches whose exchange failed
// icx_matmul_integer_noalloc's file-scope device scratch (one per GPU, for the process's life)
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
int qlinear_dql(hipStream_t s, const void* A, int a_dtype, const int8_t* Bp, int b_dtype, const int32_t* b_colsum,
                size_t M, size_t K, size_t N, const void* a_zp, const icx_chain* chain, uint8_t* y,
                float* y_scale, uint8_t* y_zp, unsigned* sync);

// icx_dynamic_quantize_linear of x [M, K] (y, y_scale, y_zp) and the quantized linear that
// reads it (icx_qlinear_f32 with A = y, its zero point y_zp, packed Int8 weight without zero
// point) as one launch, the blocks trading ranges and row-panel slices through `sync`
// (qlinear_dql's buffer and contract).  Y and the DQL outputs equal those of the two calls
// bit for bit.  K % 128 == 0, N % 96 == 0, column-only chain whose reads of y_scale are
// scalar, every block's share of its row panel within its registers (256x192 tiles, else
// 64x96), 16-byte aligned x, y and weight, a grid of at most kQoutMaxBlocks resident
// blocks; otherwise ICX_ERR_UNSUPPORTED, having launched nothing.
int dql_qlinear(hipStream_t s, const float* x, size_t M, size_t K, uint8_t* y, float* y_scale, uint8_t* y_zp,
                const int8_t* Bp, int b_dtype, const int32_t* b_colsum, size_t N, const icx_chain* chain, float* Y,
                unsigned* sync);

// Synchronise `s`, then read and clear the exchange buffer's sticky error word:
// ICX_ERR_KERNEL (with a message) if any launch since the last check gave up waiting.
int exchange_status(hipStream_t s, unsigned* sync);

// DynamicQuantizeLinear of a flat x as one launch: the blocks keep x in registers (1, 2 or
// 4 float4 per lane) and trade their (min, max) through `sync` (the layout, contract and
// failure reporting of qlinear_dql's).  Needs 16-byte aligned x, 4-byte aligned y and a grid
// of at most kQoutMaxBlocks resident blocks (n <= 4 Mi + 3); otherwise ICX_ERR_UNSUPPORTED,
// having launched nothing.  y, y_scale, y_zp equal icx_dynamic_quantize_linear's bit for bit.
int dql_exchange(hipStream_t s, const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                 unsigned* sync);

// The fault test hook of the exchange launches (icx_debug_qout_fault): 0 normally, else the
// microseconds after which a wait gives up, every wait expecting a tag nobody publishes.
int qout_fault_spin();

// How long a block of an exchange launch waits for the other blocks' ranges before it gives
// up (the launch then reports ICX_ERR_KERNEL through icx_graph_status).  A wait normally
// ends within microseconds: every block is resident and publishes right after its own work.
constexpr unsigned kExchangeWaitUs = 20000;

// `us` microseconds in ticks of the current device's wall clock (wall_clock64; the rate is
// queried once per device, 100 MHz assumed if the query fails).
inline unsigned long long wall_ticks(unsigned us) {
    static int khz[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return (unsigned long long)us * 100;
    if (!khz[dev]) {
        int r = 0;
        if (hipDeviceGetAttribute(&r, hipDeviceAttributeWallClockRate, dev) != hipSuccess || r <= 0) r = 100000;
        khz[dev] = r;
    }
    return (unsigned long long)us * (unsigned long long)khz[dev] / 1000ull;
}

// icx_dynamic_quantize_linear's two launches; `nt_y` writes a flat (no row sums) y with
// non-temporal stores (the C entry point); the graph executor passes false.
int dql_two_launch(hipStream_t s, const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                   int32_t* opt_rowsum, size_t row_len, void* ws, size_t ws_bytes, bool nt_y);

// Gather(table [axis_len, cols] UInt8 / Int8, indices) -> DequantizeLinear(., scale, zp) with a
// per-tensor scale (and zero point, may be null) in one launch: y [n_idx, cols] f32, bit for
// bit the two ops' result.  cols % 4 == 0, 4-byte aligned table, 16-byte aligned y; otherwise
// ICX_ERR_UNSUPPORTED, having launched nothing.
int gather_dequant_f32(hipStream_t s, const void* table, int dtype, size_t axis_len, size_t cols, const void* indices,
                       int idx_dtype, size_t n_idx, const float* scale, const void* zp, float* y);

// ---- layout.hip: the shape / mask plumbing of an exported encoder -----------------------
constexpr int kLayoutMaxRank = 8;
constexpr size_t kUploadMaxBytes = 64 * 1024;

// y[y_off + sum_d i_d * y_strides[d]] = x[x_off + sum_d i_d * x_strides[d]] for every index
// of `dims` (element strides, negative for a reversed walk, 0 for a broadcast dimension);
// elements of es = 1, 2, 4 or 8 bytes.  Slice, Expand and each input of Concat.
int strided_copy(hipStream_t s, const void* x, void* y, size_t es, int rank, const int64_t* dims,
                 const int64_t* x_strides, int64_t x_off, const int64_t* y_strides, int64_t y_off);

// y (dense Bool, one byte 0 / 1) = a == b over `dims`, the operands read through their own
// (broadcast) element strides; dtype: ICX_I8 / U8 / BOOL / I32 / F32 / I64.
int compare_equal(hipStream_t s, int dtype, const void* a, const int64_t* a_strides, const void* b,
                  const int64_t* b_strides, int rank, const int64_t* dims, uint8_t* y);

// out (dense) = c ? x : y over `dims`, each input read through its own (broadcast) strides;
// c is Bool (one byte, nonzero = true), x / y / out elements of es bytes.
int select_where(hipStream_t s, size_t es, const uint8_t* c, const int64_t* c_strides, const void* x,
                 const int64_t* x_strides, const void* y, const int64_t* y_strides, int rank,
                 const int64_t* dims, void* out);

// y (dense) = a op b over `dims` (op: ICX_OP_ADD / SUB / MUL / DIV), each operand read
// through its own (broadcast) strides, one IEEE f32 rounding per element.
int binary_f32(hipStream_t s, int op, const float* a, const int64_t* a_strides, const float* b,
               const int64_t* b_strides, int rank, const int64_t* dims, float* y);

// Elementwise Cast of n elements from I8 / U8 / BOOL / I32 / I64 / F32 to F32 / I64 / I32 /
// BOOL, as Rust's `as` (integers wrap or widen; to Float32 rounds to nearest even; Float32
// to an integer is NaN -> 0, saturating, else toward zero); to Bool is x != 0.
int cast_any(hipStream_t s, int src_dtype, const void* x, int dst_dtype, void* y, size_t n);

// Copy `bytes` (<= kUploadMaxBytes) of host memory to `dev` through kernel arguments: the
// host buffer may be reused as soon as this returns, and a captured graph replays the copy.
int upload_bytes(hipStream_t s, const void* host, size_t bytes, void* dev);

// DynamicQuantizeLinear of x from the n_part partials its producer left: one launch (the
// quantize pass of icx_dynamic_quantize_linear, which folds them).
int dql_from_parts(hipStream_t s, const float* x, size_t n, uint8_t* y, float* y_scale, uint8_t* y_zp,
                   int32_t* rowsum, size_t row_len, const float2* part, int n_part);

}  // namespace icx
