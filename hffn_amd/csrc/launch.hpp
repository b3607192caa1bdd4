// Host-side launchers of the HFFN kernels, shared by the translation units of the library.
// Every launcher assumes arguments already validated by the C ABI (abi.hip) and returns the
// hipError_t of its launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hffn {

enum ValueType : int { kF32 = 0, kBF16 = 1 };

constexpr uint32_t kMaxTokens = 1u << 18;  // largest n of any entry point

// Tokens per pass of the lane-per-slot ("edges") kernels: 1, 2, 4, or 8 for n > 4.
constexpr uint32_t kEdgesMaxTokens = 8;
inline uint32_t edges_tokens(uint32_t n) { return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : 8; }
// The down edges kernel stages act of its tokens in LDS up to this many bytes (else gathers it from L2): one block of
// 16 waves per CU, so the stage may take most of the CU's 160 KB. Staged by DMA with every transfer issued before one
// wait, 64-128 KB per block beat the L2 gathers (edges pair, MI355X: 410M layer at 4 / 8 tokens 15.9 -> 15.1 /
// 24.7 -> 22.7 us; 1.4B bf16 layer at 2 / 4 tokens 19.8 -> 16.6 / 25.4 -> 21.4 us).
constexpr size_t kEdgesStageBytes = 131072;

// x[rows, cols] (row stride in_ld) -> out[cols, rows] (row stride out_ld).
hipError_t launch_transpose(const float* in, float* out, uint32_t rows, uint32_t cols, uint32_t in_ld,
                            uint32_t out_ld, hipStream_t stream);

// Up projection + bias + GELU. `edges`: one wave per neuron, lanes over its slots, x token-major
// [n, d_model]; `rows`: one wave per neuron, lanes over tokens, x feature-major x_t[d_model, ld].
// Activations hidden-major act[d_ff, ld]; z (when not null) receives the pre-activation b + sum, same layout.
hipError_t launch_up_edges(int vt, const float* x, const int32_t* off, const int16_t* idx, const void* w,
                           const float* b, float* act, float* z, uint32_t d, uint32_t h, uint32_t n, uint32_t ld,
                           uint32_t nnz, hipStream_t stream);
hipError_t launch_up_rows(int vt, const float* x_t, const int32_t* off, const int16_t* idx, const void* w,
                          const float* b, float* act, float* z, uint32_t d, uint32_t h, uint32_t n, uint32_t ld,
                          hipStream_t stream);
// The rows up kernel with the backward's epilogue: gz[r, t] = (sum over the slots of r of v * gy_t[idx, t]) *
// gelu'(z[r, t]), hidden-major [h, ld] (fp32 values).
// The same with the edges up kernel (small n; gy token-major [n, d_model], its stage must fit the LDS as for the up).
hipError_t launch_grad_hidden_edges(const float* gy, const int32_t* off, const int16_t* idx, const float* v, const float* z,
                                    float* gz, uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz, hipStream_t stream);
hipError_t launch_grad_hidden_rows(const float* gy_t, const int32_t* off, const int16_t* idx, const float* v, const float* z,
                                   float* gz, uint32_t h, uint32_t n, uint32_t ld, hipStream_t stream);

// Down projection over the output-major store. `edges`: one wave per output, lanes over its
// slots, writes y[n, d_model]; `rows`: one wave per output, lanes over tokens, writes
// y_t[d_model, ld] (the caller transposes). A null bias adds nothing (the backward's gx).
hipError_t launch_down_edges(int vt, const float* act, const int32_t* off, const int16_t* hid, const void* v,
                             const float* bias, float* y, uint32_t d, uint32_t h, uint32_t n, uint32_t ld, uint32_t nnz,
                             hipStream_t stream);
// down rows: y feature-major [d, ld], or token-major [n, d] (token_major: the forward's output, no transpose after).
hipError_t launch_down_rows(int vt, const float* act, const int32_t* off, const int16_t* hid, const void* v,
                            const float* bias, float* y, uint32_t d, uint32_t n, uint32_t ld,
                            hipStream_t stream, bool token_major = false);

// Training (train.hip). Token tiles of kGradTile tokens; with more than one tile the SDDMM kernels write tile
// partials (row k of a [tiles, stride] workspace) that launch_reduce_tiles adds in tile order.
constexpr uint32_t kGradTile = 256;
inline uint32_t grad_tiles(uint32_t n) { return (n + kGradTile - 1) / kGradTile; }
// For each owner row o (rows of them) and each slot q of o: g[k*stride + q] = sum over the tokens t of tile k of
// row[o, t] * mat[idx[q], t]; gb[k*stride + o] = sum over the same tokens of row[o, t]. row and mat are [*, ld].
// n <= kEdgesMaxTokens: lanes over the slots of an owner row, the n tokens of the row in registers (one tile).
hipError_t launch_grad_sddmm_edges(const float* row, const float* mat, const int32_t* off, const int16_t* idx, float* g, float* gb,
                                   uint32_t rows, uint32_t n, uint32_t ld, hipStream_t stream);
hipError_t launch_grad_sddmm(const float* row, const float* mat, const int32_t* off, const int16_t* idx, float* g, float* gb,
                             uint32_t rows, uint32_t n, uint32_t ld, uint32_t stride, hipStream_t stream);
hipError_t launch_reduce_tiles(const float* ws, uint32_t stride, uint32_t tiles, uint32_t c1, uint32_t c2, uint32_t c3,
                               float* g_down, float* gb_down, float* g_up, float* gb_up, hipStream_t stream);
hipError_t launch_adamw(float* p, const float* g, float* m, float* v, uint32_t count, float lr_decay, float beta1,
                        float one_minus_beta1, float beta2, float one_minus_beta2, float step_size, float bias2_sqrt, float eps,
                        hipStream_t stream);
hipError_t launch_gather_values(const float* src, const int32_t* pos, float* dst, uint32_t count, hipStream_t stream);

// Output-major transpose of the hidden-major down store (stable in slot order).
uint32_t output_major_chunks(uint32_t nnz);
hipError_t launch_output_major(int vt, const int32_t* down_offsets, const int16_t* down_idx, const void* down_val,
                               uint32_t d, uint32_t h, uint32_t nnz, int32_t* out_offsets, int16_t* out_hidden,
                               void* out_val, int32_t* counts, hipStream_t stream);

// Tile-densified MFMA path (mfma.hip). Planes: fp16 hi/lo of a dense [rows, k] matrix, K-chunk-major.
// The workspace holds the split-K counters (zero between calls), the token and activation binades, the input and
// activation planes and the split-K partial sums; it must be zero-filled before its first use. The up launcher
// leaves the activations in the workspace, where the down launcher reads them.
size_t dense_plane_halves(uint32_t rows, uint32_t k);
bool mfma_shape_supported(uint32_t d, uint32_t h);
bool mfma_streamed(uint32_t n, uint32_t d, uint32_t h);  // both projections on the streamed (LDS DMA) GEMM
size_t mfma_workspace_bytes(uint32_t n, uint32_t d, uint32_t h);
hipError_t launch_densify(int vt, const int32_t* off, const int16_t* idx, const void* val, uint32_t rows, uint32_t k,
                          void* planes, int32_t* exps, hipStream_t stream);
hipError_t launch_mfma_up(int vt, const float* x, const void* planes, const int32_t* w_exp, const float* b_up, void* workspace,
                          uint32_t n, uint32_t d, uint32_t h, hipStream_t stream);  // launch_mfma_split, then launch_mfma_up_planes
hipError_t launch_mfma_split(const float* x, void* workspace, uint32_t n, uint32_t d, uint32_t h, hipStream_t stream);
hipError_t launch_mfma_up_planes(int vt, const void* planes, const int32_t* w_exp, const float* b_up, void* workspace, uint32_t n,
                                 uint32_t d, uint32_t h, hipStream_t stream);
hipError_t launch_mfma_down(int vt, const void* planes, const int32_t* v_exp, const float* b_down, float* y, void* workspace,
                            uint32_t n, uint32_t d, uint32_t h, hipStream_t stream);

// Sampled products of the training backward on the streamed GEMM (mfma.hip): the dense G = A B^T over the tokens,
// then the support's entries and the bias gradient (A [rows, ld], B [cols, ld] row-major, n real columns).
// grad_dense_workspace_bytes is 0 for shapes the streamed GEMM does not take.
size_t grad_dense_workspace_bytes(uint32_t rows, uint32_t cols, uint32_t n);
hipError_t launch_grad_dense(const float* row, const float* mat, const int32_t* off, const int16_t* idx, float* g, float* gb,
                             uint32_t rows, uint32_t cols, uint32_t n, uint32_t ld, void* workspace, hipStream_t stream);

// The training forward (z, act hidden-major; y) and the backward products gz (hidden-major) and gx on the planes
// (mfma.hip; fp32 weights): the up-shaped products as split products with the training epilogues, the down-shaped ones
// on the inference down GEMM. The workspace is the MFMA workspace with partials at every split count; both need the
// streamed GEMM (mfma_streamed).
size_t train_mfma_workspace_bytes(uint32_t n, uint32_t d, uint32_t h);
hipError_t launch_train_forward(const float* x, const void* up_planes, const int32_t* up_exp, const float* b_up, const void* down_planes,
                                const int32_t* down_exp, const float* b_down, void* workspace, float* x_t, float* act, float* z, float* y,
                                uint32_t n, uint32_t d, uint32_t h, uint32_t ld, hipStream_t stream);
hipError_t launch_train_backward(const float* gy, const float* z, const void* down_t_planes, const int32_t* down_t_exp,
                                 const void* up_t_planes, const int32_t* up_t_exp, void* workspace, float* gz, float* gx, uint32_t n,
                                 uint32_t d, uint32_t h, uint32_t ld, hipStream_t stream);

// Decode-sized projections over the same planes (gemv.hip): act token-major [n, h] (16-byte aligned), y token-major
// [n, d]; `work` (gemv_workspace_bytes) holds the k-split partial sums.
constexpr uint32_t kGemvMaxTokens = 64;
size_t gemv_workspace_bytes(uint32_t d, uint32_t h);
// The library's own k-split partials for callers that cannot allocate: a file-scope device array of
// gemv_scratch_bytes() per GPU; gemv_scratch_address gives its address on the current device (looked up once per
// device with hipGetSymbolAddress). Calls that overlap on one GPU share it and race.
size_t gemv_scratch_bytes();
hipError_t gemv_scratch_address(float** address);
hipError_t launch_gemv_forward(int vt, const float* x, const void* up_planes, const int32_t* up_exps, const float* b_up,
                               const void* down_planes, const int32_t* down_exps, const float* b_down, float* act, float* work,
                               float* y, uint32_t d, uint32_t h, uint32_t n, hipStream_t stream);

// Decode-sized projections on the tiled store (tiles.hip), 1-kTilesMaxTokens tokens; x, act and y token-major. Each
// side's tiled store (tiles_store_size: bytes of the store, int32 entries of its table; built at load by
// launch_tiles_build from the side's compact rows) holds the slots of every 16-row tile and 512-wide sub-chunk of K
// together in 8-slot groups; `work` (tiles_workspace_bytes) holds the per-chunk partial sums of a side whose blocks
// split K. tiles_shape: the block shape of a side (row tiles per block, sub-chunks per block, chunks, row blocks),
// a function of the side's shape and slot count only, so that a token's arithmetic does not depend on the call's token
// count.
constexpr uint32_t kTilesMaxTokens = 64;
struct TilesShape {
    uint32_t tr, s, chunks, blocks;
};
struct TilesStoreSize {
    uint64_t store_bytes, table_entries;
};
TilesShape tiles_shape(int vt, uint32_t rows, uint32_t K, uint64_t nnz);
TilesStoreSize tiles_store_size(int vt, uint32_t rows, uint32_t K, uint64_t nnz);
size_t tiles_workspace_bytes(int vt, uint32_t n, uint32_t d, uint32_t h, uint64_t nnz_up, uint64_t nnz_down);
// The tiles path on the compact rows: a side's table (tiles_table_entries int32, built by launch_tiles_table) holds,
// per row, the first slot of each 512-wide sub-chunk of K and the row's end, then (float32) the row's power of two.
uint64_t tiles_table_entries(int vt, uint32_t rows, uint32_t K);
hipError_t launch_tiles_table(int vt, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t K,
                              int32_t* table, hipStream_t stream);
hipError_t launch_tiles_compact(int vt, const float* x, const int16_t* up_idx, const void* up_val, const int32_t* up_table,
                                const float* b_up, const int16_t* out_hidden, const void* out_val, const int32_t* down_table,
                                const float* b_down, float* act, float* work, float* y, uint32_t d, uint32_t h, uint64_t nnz_up,
                                uint64_t nnz_down, uint32_t n, hipStream_t stream);
hipError_t launch_tiles_build(int vt, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t K, void* store,
                              int32_t* table, hipStream_t stream);
hipError_t launch_tiles_forward(int vt, const float* x, const void* up_store, const int32_t* up_table, const float* b_up,
                                const void* down_store, const int32_t* down_table, const float* b_down, float* act, float* work,
                                float* y, uint32_t d, uint32_t h, uint64_t nnz_up, uint64_t nnz_down, uint32_t n, hipStream_t stream);

// probe.hip
hipError_t launch_read_probe(const void* data, uint64_t bytes, uint32_t* sink, uint32_t blocks, hipStream_t stream);

}  // namespace hffn
