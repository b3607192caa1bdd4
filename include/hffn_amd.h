/* C ABI of the MI355X (gfx950) HFFN forward library, libhffn_amd.so.
 *
 * One fixed-support sparse FFN  y = W_down gelu(W_up x + b_up) + b_down  stored per hidden
 * neuron (compact int16 indices, float32 or bfloat16 values, float32 biases, exact-erf GELU).
 * Every pointer is a device pointer unless stated otherwise; every launch goes on `stream`
 * (a hipStream_t, NULL for the default stream) and is asynchronous. Every entry point returns
 * HFFN_OK (0) or a negative HFFN_ERROR_* code; hffn_last_error() then describes the failure
 * (per calling thread). No entry point allocates memory or synchronises.
 *
 * Layouts (n tokens, ld = leading dimension of the feature-major buffers, ld % 4 == 0, ld >= n):
 *   x      float32 [n, d_model]     token-major input
 *   x_t    float32 [d_model, ld]    feature-major input (workspace)
 *   act    float32 [d_ff, ld]       hidden-major activations gelu(z) (workspace)
 *   y_t    float32 [d_model, ld]    feature-major output (workspace)
 *   y      float32 [n, d_model]     token-major output
 *   up store:   up_offsets int32[d_ff + 1], up_idx int16[nnz_up] (input feature of each slot),
 *               up_val float32|bf16[nnz_up], b_up float32[d_ff]
 *   down store: out_offsets int32[d_model + 1], out_hidden int16[nnz_down] (hidden neuron of each
 *               slot, ascending within an output), out_val float32|bf16[nnz_down], b_down float32[d_model]
 */
#ifndef HFFN_AMD_H
#define HFFN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HFFN_ABI_VERSION 18

#define HFFN_OK 0
#define HFFN_ERROR_ARGUMENT (-1) /* invalid shape, mode, pointer or workspace */
#define HFFN_ERROR_LAUNCH (-2)   /* the HIP runtime refused a launch */

#define HFFN_VALUE_F32 0
#define HFFN_VALUE_BF16 1

/* Kernel shapes. EDGES: lanes over a row's slots in groups of consecutive slots, 16-byte value loads (fp32: 4 slots,
 * index arrays 8-byte aligned; bf16: 8 slots, index arrays 16-byte aligned; value arrays 16-byte aligned; nnz bounds
 * the grouped loads), long rows split over up to 4 waves,
 * tokens taken nt at a time (nt = 1, 2, 4 for n <= 4, else 8; ld must be a multiple of nt; the up input of nt tokens
 * is staged in LDS). ROWS: one wave per neuron/output, lanes over tokens. nnz_up / nnz_down: slots of each store. */
#define HFFN_UP_EDGES 1
#define HFFN_UP_ROWS 2
#define HFFN_DOWN_EDGES 1
#define HFFN_DOWN_ROWS 2

#define HFFN_MAX_TOKENS (1u << 18)            /* runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:26 */
#define HFFN_MAX_WIDTH 32768u                 /* widths addressable by the int16 indices */
#define HFFN_MAX_OUTPUT_MAJOR_WIDTH 16384u    /* d_model of the output-major build (LDS bins) */
#define HFFN_EDGES_MAX_LDS 131072u            /* bytes of the up input staged by the EDGES shape */

int hffn_abi_version(void);
const char* hffn_last_error(void);

/* 1 if the EDGES up shape can stage n tokens of width d_model in LDS, else 0 (host-only query). */
int hffn_edges_supported(uint32_t d_model, uint32_t n);

/* out[c, r] = in[r, c] for r < rows, c < cols (row strides in_ld and out_ld, in floats).
 * Replaces the `x_t.copy_(x.T)` of runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:150-151. */
int hffn_transpose(const float* in, float* out, uint32_t rows, uint32_t cols, uint32_t in_ld, uint32_t out_ld,
                   void* stream);

/* act[r, t] = gelu(b_up[r] + sum_{e in [up_offsets[r], up_offsets[r+1])} up_val[e] * x[t, up_idx[e]]).
 * mode EDGES reads x token-major [n, d_model]; mode ROWS reads x feature-major [d_model, ld].
 * Replaces the up kernels `up_coop` / `up_lane` / `up_tile(const float* x, const int* off,
 * const short* idx, const float* w, const float* b, float* a, unsigned d, unsigned H, unsigned n)`
 * of runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py:102-143 (launch: runtime.py:143-155). */
int hffn_up(int mode, int value_type, const float* x, const int32_t* up_offsets, const int16_t* up_idx,
            const void* up_val, const float* b_up, float* act, uint32_t d_model, uint32_t d_ff, uint32_t nnz_up, uint32_t n,
            uint32_t ld, void* stream);

/* y[t, o] = sum_{q in [out_offsets[o], out_offsets[o+1])} out_val[q] * act[out_hidden[q], t] + b_down[o].
 * mode EDGES writes y token-major [n, d_model]; mode ROWS writes y feature-major [d_model, ld].
 * Replaces `down_coop` / `down_tiled` / `down_blocked(const float* a, const int* off, const short* hid,
 * const float* v, const float* bias, float* y, unsigned d, unsigned n)` of
 * runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py:145-191 (launch: runtime.py:156-162). */
int hffn_down(int mode, int value_type, const float* act, const int32_t* out_offsets, const int16_t* out_hidden,
              const void* out_val, const float* b_down, float* y, uint32_t d_model, uint32_t d_ff, uint32_t nnz_down,
              uint32_t n, uint32_t ld, void* stream);

/* The whole layer for x[n, d_model] -> y[n, d_model]: the transposes the modes need, up, down.
 * x_t may be NULL when the up mode is not ROWS; y_t is not written (the ROWS down kernel writes y token-major itself)
 * and may be NULL. act is a workspace here: for one or two tokens on the
 * EDGES/EDGES pair it holds the activations packed [d_ff, n] (its first n d_ff floats). Replaces HFFNRuntime._launch
 * (runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:134-163). */
int hffn_forward(int up_mode, int down_mode, int value_type, const float* x, const int32_t* up_offsets,
                 const int16_t* up_idx, const void* up_val, const float* b_up, const int32_t* out_offsets,
                 const int16_t* out_hidden, const void* out_val, const float* b_down, float* x_t, float* act,
                 float* y_t, float* y, uint32_t d_model, uint32_t d_ff, uint32_t nnz_up, uint32_t nnz_down, uint32_t n,
                 uint32_t ld, void* stream);

/* Prepared forward (the decode launch path). hffn_plan_forward checks every argument of hffn_forward but x and
 * the stream, as hffn_forward does, and keeps them under a new nonzero handle *plan; hffn_plan_launch(plan, x,
 * stream) then launches that forward for x (launch errors only); hffn_plan_release drops the handle. The pointers
 * are kept as given: a plan must be released before any of its buffers is freed or reallocated. Handles are
 * process-wide and the table is locked, so plans may be made and launched from several threads. Replaces the
 * per-(layer, N) _Descriptor of PreparedRuntime (pre-packed driver argument tables, x patched per call) and its two
 * driver launches: runtime/gpu/nvidia/llm/inference/hffn_pythia_cuda/prepared_runtime.py:34-82. */
int hffn_plan_forward(int up_mode, int down_mode, int value_type, const int32_t* up_offsets, const int16_t* up_idx,
                      const void* up_val, const float* b_up, const int32_t* out_offsets, const int16_t* out_hidden,
                      const void* out_val, const float* b_down, float* x_t, float* act, float* y_t, float* y, uint32_t d_model,
                      uint32_t d_ff, uint32_t nnz_up, uint32_t nnz_down, uint32_t n, uint32_t ld, uint64_t* plan);
int hffn_plan_launch(uint64_t plan, const float* x, void* stream);
int hffn_plan_release(uint64_t plan);

/* Bytes of device workspace hffn_output_major needs for nnz down slots (host-only query). */
int hffn_output_major_workspace(uint32_t nnz, uint32_t d_model, uint64_t* bytes);

/* Output-major transpose of the hidden-major down store, stable in slot order:
 *   out_offsets = [0, cumsum(bincount(down_idx, d_model))],
 *   out_hidden[p] = owner neuron of slot order[p], out_val[p] = down_val[order[p]],
 * with order = the stable argsort of down_idx. Replaces HFFNLayer.from_hidden_major
 * (runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:55-67), which runs it on the host. */
int hffn_output_major(int value_type, const int32_t* down_offsets, const int16_t* down_idx, const void* down_val,
                      uint32_t d_model, uint32_t d_ff, uint32_t nnz, int32_t* out_offsets, int16_t* out_hidden,
                      void* out_val, void* workspace, uint64_t workspace_bytes, void* stream);

/* ---- Tile-densified MFMA path (high density, large n). No reference counterpart: the reference runs every shape on
 * the gather kernels (runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py). Every operand is a pair of fp16 hi/lo
 * "planes" scaled by powers of two (binades): the weights are densified at load (one binade per row); x is split
 * before the up GEMM (one binade per token); the activations are split by the up GEMM (one binade per token and
 * 128-neuron block) and stay in the workspace. Each product is hi*hi + hi*lo + lo*hi (hi*hi + lo*hi for bf16
 * weights) on v_mfma_f32_32x32x16_f16 with fp32 accumulation; the binades are undone exactly. */

/* 1 if the MFMA path takes this shape (d_model and d_ff multiples of 256), else 0 (host-only query). */
int hffn_mfma_supported(uint32_t d_model, uint32_t d_ff);

/* 1 if both projections of n tokens run on the streamed GEMM (256 x 128 tiles whose k-tiles are transferred straight
 * into LDS, enough blocks with the k split to fill the chip), 0 if one of them falls back to the register-staged GEMM
 * (narrow layers at small n); negative on an unsupported shape. Host-only query. No counterpart in the reference,
 * whose policy (runtime.py:29-39) has no densified path; the runtime's policy takes the MFMA path only when this is 1. */
int hffn_mfma_streamed(uint32_t n, uint32_t d_model, uint32_t d_ff);

/* Bytes of the planes of a dense [rows, k] matrix (host-only query). */
int hffn_dense_planes_bytes(uint32_t rows, uint32_t k, uint64_t* bytes);

/* Densify one side: row r holds slots [offsets[r], offsets[r+1]) at columns idx[] (distinct within a row, in [0, k)).
 * The up side is rows = d_ff over k = d_model from (up_offsets, up_idx, up_val); the down side is rows = d_model over
 * k = d_ff from the output-major (out_offsets, out_hidden, out_val). Writes every byte of `planes` and binades[rows]. */
int hffn_densify(int value_type, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t k,
                 void* planes, int32_t* binades, void* stream);

/* Bytes of the device workspace of the MFMA entry points for n tokens (host-only query; the entry points refuse a
 * smaller workspace_bytes). The workspace holds one
 * counter per output tile of the down projection, the token and activation binades, the planes of x and of the
 * activations (n padded to 256 rows) and the split-K partial sums; it must be zero-filled before its first use, and
 * every call leaves the counters at zero. Calls that share a workspace must be ordered (one stream). */
int hffn_mfma_workspace(uint32_t n, uint32_t d_model, uint32_t d_ff, uint64_t* bytes);

/* act[t, r] = gelu(b_up[r] + sum_i W_up[r, i] x[t, i]), left in the workspace as planes with one binade per token and
 * 128-neuron block (read by hffn_mfma_down); also splits x (16-byte aligned) into the workspace. */
int hffn_mfma_up(int value_type, const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up,
                 void* workspace, uint64_t workspace_bytes, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream);

/* The two halves of hffn_mfma_up, for callers that time or reuse them apart (no reference counterpart):
 * hffn_mfma_split splits x (16-byte aligned) into the workspace's token planes and binades; hffn_mfma_up_planes runs
 * the up GEMM on them (act as hffn_mfma_up leaves it). hffn_mfma_up = hffn_mfma_split, then hffn_mfma_up_planes. */
int hffn_mfma_split(const float* x, void* workspace, uint64_t workspace_bytes, uint32_t d_model, uint32_t d_ff, uint32_t n,
                    void* stream);
int hffn_mfma_up_planes(int value_type, const void* up_planes, const int32_t* up_binades, const float* b_up, void* workspace,
                        uint64_t workspace_bytes, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream);

/* y[t, o] = sum_r W_down[o, r] act[t, r] + b_down[o], y token-major [n, d_model]; the activations as left in the
 * workspace by hffn_mfma_up for the same n. */
int hffn_mfma_down(int value_type, const void* down_planes, const int32_t* down_binades, const float* b_down, float* y,
                   void* workspace, uint64_t workspace_bytes, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream);

/* The whole layer on the MFMA path (hffn_mfma_up then hffn_mfma_down). */
int hffn_forward_mfma(int value_type, const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up,
                      const void* down_planes, const int32_t* down_binades, const float* b_down, void* workspace,
                      uint64_t workspace_bytes, float* y, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream);

/* ---- Decode path on the planes (1-64 tokens). No reference counterpart: the reference decodes on its gather kernels
 * (runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py). One kernel per projection reads the planes once as
 * whole lines and multiplies on v_mfma_f32_16x16x32_f16 (tokens padded to 16, 32 or 64). */

/* Bytes of the device workspace of hffn_forward_gemv (host-only query; the same for every n): the k-split partial sums
 * of a projection whose 16-row tiles alone leave CUs idle (added by a second, small kernel). No initial contents are
 * needed. Calls that share a workspace must be ordered (one stream). */
int hffn_gemv_workspace(uint32_t d_model, uint32_t d_ff, uint64_t* bytes);

/* act[t, r] = gelu(b_up[r] + sum_i W_up[r, i] x[t, i]) into act (token-major [n, d_ff], 16-byte aligned, like x),
 * then y[t, o] = b_down[o] + sum_r W_down[o, r] act[t, r] (token-major [n, d_model]); 1 <= n <= 64. The inputs are
 * split into fp16 hi/lo with one power of two per token and 32-k tile, the products summed as on the MFMA path.
 * Every output is a fixed-order sum, independent of the other tokens of the call. */
int hffn_forward_gemv(int value_type, const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up,
                      const void* down_planes, const int32_t* down_binades, const float* b_down, float* act, void* workspace,
                      uint64_t workspace_bytes, float* y, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream);

/* hffn_forward_gemv without a workspace argument, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. The k-split partial
 * sums go to the library's own static device array (HFFN_GEMV_STATIC_SCRATCH_BYTES per GPU, held until the process
 * ends; its address on the current device is looked up once per device); shapes needing more are refused with
 * HFFN_ERROR_ARGUMENT, and no call allocates or frees anything. The partials need no initial contents. Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (several streams or threads) race. */
#define HFFN_GEMV_STATIC_SCRATCH_BYTES (1u << 20)
int hffn_forward_gemv_static(int value_type, const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up,
                             const void* down_planes, const int32_t* down_binades, const float* b_down, float* act, float* y,
                             uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream);

/* Prepared decode-GEMV forward: checks every argument of hffn_forward_gemv but x and the stream and keeps them under a
 * new nonzero handle, launched by hffn_plan_launch (which then checks x's alignment) and dropped by hffn_plan_release,
 * like hffn_plan_forward's. No reference counterpart beyond the prepared descriptors that plan_forward mirrors
 * (prepared_runtime.py:34-82): this is the same launch path for the decode GEMVs. */
int hffn_plan_gemv(int value_type, const void* up_planes, const int32_t* up_binades, const float* b_up, const void* down_planes,
                   const int32_t* down_binades, const float* b_down, float* act, void* workspace, uint64_t workspace_bytes, float* y,
                   uint32_t d_model, uint32_t d_ff, uint32_t n, uint64_t* plan);

/* ---- Decode path on the compact store (1-64 tokens). No reference counterpart for the arithmetic: the reference
 * decodes on its gather kernels (runtime/gpu/nvidia/common/kernels/hffn_cuda/kernels.py:102-191), reading each slot
 * once per kernel as these do. Each side is read from its tiled store: a copy of the side's compact rows, built once at
 * load, in which the slots of every 16-row tile and 512-wide sub-chunk of K (an item) are consecutive, in 8-slot groups
 * of interleaved 16-bit fields ([8 positions][8 bfloat16 weights], 32 bytes; or [8 positions][8 fp16 hi][8 fp16 lo],
 * 48 bytes, hi + lo = the float32 weight scaled by the power of two of its row's largest |weight|), each item padded
 * to whole groups with its last slot repeated. A block reads the groups of 16 or 32 rows over a chunk of K (16-byte
 * loads, each slot once per call), densifies them in LDS and multiplies on 16x16x32 MFMAs (float32: x split per token
 * into fp16 hi/lo, three products; bfloat16: x split exactly into three bfloat16 parts). Sides whose blocks split K
 * write per-chunk partials, added in chunk order by a second kernel. x, act and y token-major; x and act 16-byte
 * aligned. */

/* Sizes of one side's tiled store for nnz slots over rows x k (host-only query): bytes of the store (an upper bound:
 * padding of at most one group per item, one spare group) and int32 entries of its table (items + 1, then one per row
 * for float32 values; items = ceil(rows / 16) * ceil(k / 512)). */
int hffn_tiles_store_size(int value_type, uint32_t rows, uint32_t k, uint64_t nnz, uint64_t* store_bytes, uint64_t* table_entries);

/* Builds one side's tiled store and table on the device, once at load: the up side from (up_offsets, up_idx, up_val,
 * rows = d_ff, k = d_model), the down side from (out_offsets, out_hidden, out_val, rows = d_model, k = d_ff). Every
 * row's indices must be strictly increasing and below k. table[i] = the first group of item i (items of tile t and
 * sub-chunk j at i = t * ceil(k / 512) + j), table[items] = the number of groups, then (float32) the rows' powers of
 * two. store 16-byte aligned, of at least the bytes hffn_tiles_store_size gives. */
int hffn_tiles_build(int value_type, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t k,
                     uint64_t nnz, void* store, uint64_t store_bytes, int32_t* table, void* stream);

/* Bytes of the workspace of hffn_forward_tiles for n tokens (host-only query): the per-chunk partials of a side whose
 * blocks split K. The block shape of each side depends on its dimensions and slot count (nnz_up, nnz_down), never on n.
 * No initial contents needed; calls that share it must be ordered (one stream). */
int hffn_tiles_workspace(int value_type, uint32_t n, uint32_t d_model, uint32_t d_ff, uint64_t nnz_up, uint64_t nnz_down,
                         uint64_t* bytes);

/* act[t, r] = gelu(b_up[r] + sum_k W_up[r, k] x[t, k]) into act (token-major [n, d_ff]), then
 * y[t, o] = b_down[o] + sum_r W_down[o, r] act[t, r] (token-major [n, d_model]); 1 <= n <= 64, d_model a multiple of
 * 16, d_ff of 8. The stores and tables are hffn_tiles_build's of the two sides, over nnz_up and nnz_down slots. */
int hffn_forward_tiles(int value_type, const float* x, const void* up_store, const int32_t* up_table, const float* b_up,
                       const void* down_store, const int32_t* down_table, const float* b_down, float* act, void* workspace,
                       uint64_t workspace_bytes, float* y, uint32_t d_model, uint32_t d_ff, uint64_t nnz_up, uint64_t nnz_down,
                       uint32_t n, void* stream);

/* Prepared hffn_forward_tiles (every argument but x and the stream checked and kept under a handle), launched by
 * hffn_plan_launch and dropped by hffn_plan_release as hffn_plan_forward's: the decode launch path of
 * PreparedRuntime (runtime/gpu/nvidia/llm/inference/hffn_pythia_cuda/prepared_runtime.py:34-82) for this path. */
int hffn_plan_tiles(int value_type, const void* up_store, const int32_t* up_table, const float* b_up, const void* down_store,
                    const int32_t* down_table, const float* b_down, float* act, void* workspace, uint64_t workspace_bytes, float* y,
                    uint32_t d_model, uint32_t d_ff, uint64_t nnz_up, uint64_t nnz_down, uint32_t n, uint64_t* plan);

/* The tiles path on the compact rows themselves (no tiled copy: the layer's only resident store), the same products
 * and the same bits as hffn_forward_tiles, the tiles read by per-row ranges of 8-slot pieces (16-byte loads of the
 * index and value arrays). A side's table (hffn_tiles_table_size int32 entries, built by hffn_tiles_table_build from its
 * compact rows) holds, per row, the first slot of each 512-wide sub-chunk of k and the row's end, then (float32) each
 * row's power of two. The index and value arrays must be 16-byte aligned; the rest as hffn_forward_tiles.
 * hffn_plan_tiles_compact keeps every argument but x and the stream under a plan handle (hffn_plan_launch). */
int hffn_tiles_table_size(int value_type, uint32_t rows, uint32_t k, uint64_t* entries);
int hffn_tiles_table_build(int value_type, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t k,
                           int32_t* table, void* stream);
int hffn_forward_tiles_compact(int value_type, const float* x, const int16_t* up_idx, const void* up_val, const int32_t* up_table,
                               const float* b_up, const int16_t* out_hidden, const void* out_val, const int32_t* down_table,
                               const float* b_down, float* act, void* workspace, uint64_t workspace_bytes, float* y, uint32_t d_model,
                               uint32_t d_ff, uint64_t nnz_up, uint64_t nnz_down, uint32_t n, void* stream);
int hffn_plan_tiles_compact(int value_type, const int16_t* up_idx, const void* up_val, const int32_t* up_table, const float* b_up,
                            const int16_t* out_hidden, const void* out_val, const int32_t* down_table, const float* b_down, float* act,
                            void* workspace, uint64_t workspace_bytes, float* y, uint32_t d_model, uint32_t d_ff, uint64_t nnz_up,
                            uint64_t nnz_down, uint32_t n, uint64_t* plan);

/* ------------------------------------------------------------------------------------------------ training (fp32)
 * Layouts: act, z, gz hidden-major [d_ff, ld]; x_t, gy_t, gx_t feature-major [d_model, ld]; x, y, gx token-major
 * [n, d_model]. Gradients of the compact arrays in their own orders: g_up as up_val (hidden-major slots), g_down as
 * out_val (output-major edges). Token tiles of 256: for n > 256 the two sampled products write tile partials that
 * hffn_reduce_tiles adds in tile order. Every result is written by one lane: same bits run to run. */

/* hffn_forward (gather modes, fp32 values) that also writes the pre-activations z = b_up + W_up x (hidden-major, as
 * act) and x_t = x transposed for every mode. Replaces the forward of HFFNTrainRuntime.forward with a z buffer
 * (runtime/gpu/nvidia/ffn/training/train_runtime.py:133-152: the up_<mode>_z kernels of forward_source(store_z=True),
 * kernels_train.py:263). */
int hffn_forward_z(int up_mode, int down_mode, const float* x, const int32_t* up_offsets, const int16_t* up_idx, const float* up_val,
                   const float* b_up, const int32_t* out_offsets, const int16_t* out_hidden, const float* out_val, const float* b_down,
                   float* x_t, float* act, float* y_t, float* y, float* z, uint32_t d_model, uint32_t d_ff, uint32_t nnz_up,
                   uint32_t nnz_down, uint32_t n, uint32_t ld, void* stream);

/* The two sampled products of hffn_grad_sddmm (same g, gb and slot orders; no tile partials) from a dense product
 * on the streamed MFMA GEMM: G[rows, cols] = row[rows, :n] mat[cols, :n]^T with both operands split into fp16 hi/lo
 * (one power of two per row; hi*hi + hi*lo + lo*hi in fp32), then g[q] = G[o, index[q]] for the slots of each owner
 * row o, and gb[o] = sum_t row[o, t]. row and mat row-major with stride ld (16-byte aligned); rows a multiple of 256,
 * cols of 128. hffn_grad_dense_workspace refuses shapes the streamed GEMM does not take (too few tiles). No reference
 * counterpart (the reference's sampled products are gathers, kernels_train.py:115-184); for high density and many
 * tokens, where a gather reads nnz * n * 4 bytes of activations per product. */
int hffn_grad_dense_workspace(uint32_t rows, uint32_t cols, uint32_t n, uint64_t* bytes);
int hffn_grad_dense(const float* row, const float* mat, const int32_t* offsets, const int16_t* index, float* g, float* gb,
                    uint32_t rows, uint32_t cols, uint32_t n, uint32_t ld, void* workspace, uint64_t workspace_bytes, void* stream);

/* The training step's dense products on the planes (fp32 values; layers whose planes the runtime holds), for the
 * token counts the streamed GEMM takes (hffn_train_mfma_workspace refuses the others). hffn_forward_mfma_z: the forward
 * with z of hffn_forward_z on the planes of W_up [d_ff, d_model] and W_down [d_model, d_ff] (hffn_densify):
 * z = b_up + W_up x and act = gelu(z) hidden-major [d_ff, ld], x_t = x transposed, y = W_down act + b_down.
 * hffn_backward_mfma: gz = (gy W_down) * gelu'(z) hidden-major and gx = gz W_up [n, d_model], on the planes of
 * W_down^T [d_ff rows, d_model k] and W_up^T [d_model rows, d_ff k] (hffn_densify of the hidden-major down support and
 * of the input-major up support, with the values gathered into those orders). Every product is split fp16 on MFMA
 * (hi*hi + hi*lo + lo*hi, fp32 accumulation); every result is written by one lane. Float buffers 16-byte aligned, the
 * workspace (hffn_train_mfma_workspace bytes) 256-byte aligned; it holds the token planes and split partials, and the
 * calls that share it must be ordered. No reference counterpart: the reference's training kernels are gathers
 * (kernels_train.py:101-231); these replace the forward with z, grad_hidden and grad_x at high density and many tokens. */
int hffn_train_mfma_workspace(uint32_t n, uint32_t d_model, uint32_t d_ff, uint64_t* bytes);
int hffn_forward_mfma_z(const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up, const void* down_planes,
                        const int32_t* down_binades, const float* b_down, void* workspace, uint64_t workspace_bytes, float* x_t,
                        float* act, float* z, float* y, uint32_t d_model, uint32_t d_ff, uint32_t n, uint32_t ld, void* stream);
int hffn_backward_mfma(const float* gy, const float* z, const void* down_t_planes, const int32_t* down_t_binades, const void* up_t_planes,
                       const int32_t* up_t_binades, void* workspace, uint64_t workspace_bytes, float* gz, float* gx, uint32_t d_model,
                       uint32_t d_ff, uint32_t n, uint32_t ld, void* stream);

/* Sampled product over an owner-row support: for each owner o < rows, token tile k and slot q of o,
 * g[k*stride + q] = sum_t row[o, t] mat[index[q], t] and gb[k*stride + o] = sum_t row[o, t] (t over tile k, below n);
 * row, mat 16-byte aligned [*, ld]; stride is ignored for n <= 256 (the results are the gradients). With
 * row = gy_t, mat = act over the output-major down edges: g_down, gb_down; with row = gz, mat = x_t over the up
 * slots: g_up, gb_up. Replaces grad_down and grad_up (runtime/gpu/nvidia/ffn/training/kernels_train.py:115-137,
 * 162-184). */
int hffn_grad_sddmm(const float* row, const float* mat, const int32_t* offsets, const int16_t* index, float* g, float* gb,
                    uint32_t rows, uint32_t n, uint32_t ld, uint32_t stride, void* stream);

/* gz[r, t] = (sum over the hidden-major down slots of r of down_val * gy[t, down_idx]) * gelu'(z[r, t]); down_val in
 * hidden-major slot order; gy token-major (read up to 8 tokens) and gy_t feature-major (read above). Replaces
 * grad_hidden (kernels_train.py:139-160). */
int hffn_grad_hidden(const float* gy, const float* gy_t, const float* z, const int32_t* down_offsets, const int16_t* down_idx,
                     const float* down_val, float* gz, uint32_t d_model, uint32_t d_ff, uint32_t nnz_down, uint32_t n, uint32_t ld,
                     void* stream);

/* gx[t, i] = sum over the input-major up slots of i of in_val * gz[in_hidden, t] (above 8 tokens through gx_t,
 * feature-major). Replaces grad_x (kernels_train.py:201-231). */
int hffn_grad_x(const float* gz, const int32_t* in_offsets, const int16_t* in_hidden, const float* in_val, float* gx_t, float* gx,
                uint32_t d_model, uint32_t d_ff, uint32_t nnz_up, uint32_t n, uint32_t ld, void* stream);

/* Fixed-order sum of the tile partials ws[tiles, stride] into g_down [0, c1), gb_down [c1, c2), g_up [c2, c3),
 * gb_up [c3, stride). Replaces reduce_tiles (kernels_train.py:186-199). */
int hffn_reduce_tiles(const float* ws, uint32_t stride, uint32_t tiles, uint32_t c1, uint32_t c2, uint32_t c3, float* g_down,
                      float* gb_down, float* g_up, float* gb_up, void* stream);

/* Compact AdamW on one array: p -= lr_decay p; m = beta1 m + (1 - beta1) g; v = beta2 v + (1 - beta2) g^2;
 * p -= step_size m / (sqrt(v) / bias2_sqrt + eps). Replaces adamw (kernels_train.py:233-247). */
int hffn_adamw(float* p, const float* g, float* m, float* v, uint32_t count, float lr_decay, float beta1, float one_minus_beta1,
               float beta2, float one_minus_beta2, float step_size, float bias2_sqrt, float eps, void* stream);

/* dst[j] = src[pos[j]]: the values of a transposed support refreshed from the compact array they index (the
 * reference reads them through the positions inside its kernels, kernels_train.py:142-150, 204-215). */
int hffn_gather_values(const float* src, const int32_t* pos, float* dst, uint32_t count, void* stream);

/* Measurement only, no counterpart in the reference: a plain streaming read of `bytes` (a nonzero multiple of 16 from
 * a 16-byte aligned pointer) by `blocks` blocks of 4 waves, each wave one contiguous span, one word per wave written to
 * sink (sink_words >= 4 blocks). The floor that the decode calls are measured against (bench.py's decode record). */
int hffn_read_probe(const void* data, uint64_t bytes, uint32_t* sink, uint32_t sink_words, uint32_t blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HFFN_AMD_H */
