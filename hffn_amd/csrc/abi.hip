// C ABI of the HFFN HIP library: plain pointers, sizes and a hipStream_t, a status code per call
// and a per-thread message for the last failure. Declarations, and the reference interfaces each
// entry point replaces, are in include/hffn_amd.h.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <initializer_list>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/hffn_amd.h"
#include "launch.hpp"

namespace {

thread_local std::string g_error;

int fail(int code, const char* format, ...) {
    char buffer[512];
    va_list args;
    va_start(args, format);
    std::vsnprintf(buffer, sizeof(buffer), format, args);
    va_end(args);
    g_error = buffer;
    return code;
}

int launched(hipError_t status, const char* what) {
    if (status != hipSuccess) return fail(HFFN_ERROR_LAUNCH, "%s: %s", what, hipGetErrorString(status));
    return HFFN_OK;
}

bool valid_value_type(int vt) { return vt == HFFN_VALUE_F32 || vt == HFFN_VALUE_BF16; }

// Shapes shared by every forward entry: d_model a multiple of 16 (as the reference runtime requires),
// both widths addressable by the 16-bit indices, 1 <= n <= HFFN_MAX_TOKENS, ld a multiple of 4 covering n.
int check_shape(uint32_t d, uint32_t h, uint32_t n, uint32_t ld) {
    if (d == 0 || d % 16 != 0 || d > HFFN_MAX_WIDTH) return fail(HFFN_ERROR_ARGUMENT, "d_model=%u: must be a positive multiple of 16, at most %u", d, HFFN_MAX_WIDTH);
    if (h == 0 || h > HFFN_MAX_WIDTH) return fail(HFFN_ERROR_ARGUMENT, "d_ff=%u: must be in [1, %u]", h, HFFN_MAX_WIDTH);
    if (n == 0 || n > HFFN_MAX_TOKENS) return fail(HFFN_ERROR_ARGUMENT, "n=%u: unsupported token count", n);
    if (ld < n || ld % 4 != 0) return fail(HFFN_ERROR_ARGUMENT, "ld=%u: must be a multiple of 4 and at least n=%u", ld, n);
    return HFFN_OK;
}

// EDGES takes its tokens nt at a time: ld must be a multiple of nt, and the up input stage
// nt * d_model floats must fit the LDS budget.
int check_edges(uint32_t d, uint32_t n, uint32_t ld, bool stage) {
    const uint32_t nt = hffn::edges_tokens(n);
    if (ld % nt != 0) return fail(HFFN_ERROR_ARGUMENT, "edges mode: ld=%u must be a multiple of %u for n=%u", ld, nt, n);
    if (stage && static_cast<size_t>(nt) * (d + 16) * sizeof(float) > HFFN_EDGES_MAX_LDS)
        return fail(HFFN_ERROR_ARGUMENT, "edges mode: %u tokens of d_model=%u exceed the %u-byte LDS stage", nt, d, HFFN_EDGES_MAX_LDS);
    return HFFN_OK;
}

}  // namespace

extern "C" {

int hffn_abi_version(void) { return HFFN_ABI_VERSION; }

const char* hffn_last_error(void) { return g_error.c_str(); }

int hffn_edges_supported(uint32_t d_model, uint32_t n) {
    if (n == 0) return 0;
    return static_cast<size_t>(hffn::edges_tokens(n)) * (d_model + 16) * sizeof(float) <= HFFN_EDGES_MAX_LDS ? 1 : 0;
}

int hffn_transpose(const float* in, float* out, uint32_t rows, uint32_t cols, uint32_t in_ld, uint32_t out_ld,
                   void* stream) {
    if (!in || !out) return fail(HFFN_ERROR_ARGUMENT, "transpose: null pointer");
    if (rows == 0 || cols == 0) return HFFN_OK;
    if (in_ld < cols || out_ld < rows) return fail(HFFN_ERROR_ARGUMENT, "transpose: strides %u/%u smaller than %ux%u", in_ld, out_ld, rows, cols);
    return launched(hffn::launch_transpose(in, out, rows, cols, in_ld, out_ld, static_cast<hipStream_t>(stream)), "transpose");
}

namespace {
// The edges kernels read groups of slots in 16-byte value loads: float32 4 slots (8-byte index loads), bfloat16 8
// slots (16-byte index loads).
int check_store_alignment(const int16_t* idx, const void* val, int value_type) {
    const uintptr_t index_align = value_type == HFFN_VALUE_BF16 ? 16 : 8;
    if (reinterpret_cast<uintptr_t>(idx) % index_align != 0 || reinterpret_cast<uintptr_t>(val) % 16 != 0)
        return fail(HFFN_ERROR_ARGUMENT, "edges mode: index/value arrays must be %u/16-byte aligned", static_cast<unsigned>(index_align));
    return HFFN_OK;
}
}  // namespace

}  // extern "C"

namespace {

// Argument checks of hffn_up / hffn_down (everything a launch relies on), apart from the launch itself.
int check_up(int mode, int value_type, const float* x, const int32_t* up_offsets, const int16_t* up_idx, const void* up_val,
             const float* b_up, const float* act, uint32_t d_model, uint32_t d_ff, uint32_t n, uint32_t ld) {
    if (int status = check_shape(d_model, d_ff, n, ld)) return status;
    if (!valid_value_type(value_type)) return fail(HFFN_ERROR_ARGUMENT, "unknown value type %d", value_type);
    if (!x || !up_offsets || !up_idx || !up_val || !b_up || !act) return fail(HFFN_ERROR_ARGUMENT, "up: null pointer");
    if (mode == HFFN_UP_EDGES) {
        if (int status = check_edges(d_model, n, ld, true)) return status;
        return check_store_alignment(up_idx, up_val, value_type);
    }
    if (mode == HFFN_UP_ROWS) return HFFN_OK;
    return fail(HFFN_ERROR_ARGUMENT, "unknown up mode %d", mode);
}

int check_down(int mode, int value_type, const float* act, const int32_t* out_offsets, const int16_t* out_hidden,
               const void* out_val, const float* b_down, const float* y, uint32_t d_model, uint32_t d_ff, uint32_t n, uint32_t ld) {
    if (int status = check_shape(d_model, d_ff, n, ld)) return status;
    if (!valid_value_type(value_type)) return fail(HFFN_ERROR_ARGUMENT, "unknown value type %d", value_type);
    if (!act || !out_offsets || !out_hidden || !out_val || !b_down || !y) return fail(HFFN_ERROR_ARGUMENT, "down: null pointer");
    if (mode == HFFN_DOWN_EDGES) {
        if (int status = check_edges(d_model, n, ld, false)) return status;
        return check_store_alignment(out_hidden, out_val, value_type);
    }
    if (mode == HFFN_DOWN_ROWS) return HFFN_OK;
    return fail(HFFN_ERROR_ARGUMENT, "unknown down mode %d", mode);
}

int launch_up(int mode, int value_type, const float* x, const int32_t* up_offsets, const int16_t* up_idx, const void* up_val,
              const float* b_up, float* act, uint32_t d_model, uint32_t d_ff, uint32_t nnz_up, uint32_t n, uint32_t ld, hipStream_t s,
              float* z = nullptr) {
    if (mode == HFFN_UP_EDGES)
        return launched(hffn::launch_up_edges(value_type, x, up_offsets, up_idx, up_val, b_up, act, z, d_model, d_ff, n, ld, nnz_up, s),
                        "up edges");
    return launched(hffn::launch_up_rows(value_type, x, up_offsets, up_idx, up_val, b_up, act, z, d_model, d_ff, n, ld, s), "up rows");
}

int launch_down(int mode, int value_type, const float* act, const int32_t* out_offsets, const int16_t* out_hidden,
                const void* out_val, const float* b_down, float* y, uint32_t d_model, uint32_t d_ff, uint32_t nnz_down, uint32_t n,
                uint32_t ld, hipStream_t s) {
    if (mode == HFFN_DOWN_EDGES)
        return launched(hffn::launch_down_edges(value_type, act, out_offsets, out_hidden, out_val, b_down, y, d_model, d_ff, n, ld,
                                                nnz_down, s),
                        "down edges");
    return launched(hffn::launch_down_rows(value_type, act, out_offsets, out_hidden, out_val, b_down, y, d_model, n, ld, s), "down rows");
}

// Everything of one gather-mode forward but x and the stream.
struct Plan {
    int up_mode, down_mode, value_type;
    const int32_t* up_offsets;
    const int16_t* up_idx;
    const void* up_val;
    const float* b_up;
    const int32_t* out_offsets;
    const int16_t* out_hidden;
    const void* out_val;
    const float* b_down;
    float *x_t, *act, *y_t, *y;
    uint32_t d_model, d_ff, nnz_up, nnz_down, n, ld;
};

// The checks of hffn_forward with a stand-in for x (checked at each launch instead).
int check_forward(const Plan& p) {
    const float* some_x = reinterpret_cast<const float*>(uintptr_t{16});  // non-null, aligned: never dereferenced
    if (p.up_mode == HFFN_UP_ROWS && !p.x_t) return fail(HFFN_ERROR_ARGUMENT, "forward: null x_t workspace");
    const float* up_in = p.up_mode == HFFN_UP_ROWS ? p.x_t : some_x;
    if (int status = check_up(p.up_mode, p.value_type, up_in, p.up_offsets, p.up_idx, p.up_val, p.b_up, p.act, p.d_model, p.d_ff,
                              p.n, p.ld))
        return status;
    return check_down(p.down_mode, p.value_type, p.act, p.out_offsets, p.out_hidden, p.out_val, p.b_down, p.y, p.d_model, p.d_ff,
                      p.n, p.ld);
}

// hffn_forward after its checks. With z (the training forward) the pre-activations go to z and x_t is written for
// every mode (the backward reads x feature-major).
int launch_forward(const Plan& p, const float* x, hipStream_t s, float* z = nullptr) {
    if (p.up_mode == HFFN_UP_ROWS || z) {
        if (int status = launched(hffn::launch_transpose(x, p.x_t, p.n, p.d_model, p.d_model, p.ld, s), "input transpose")) return status;
    }
    if (p.up_mode == HFFN_UP_ROWS) x = p.x_t;
    // One or two tokens on the lane-per-slot pair (without z): the activations are packed [d_ff, n] in the workspace,
    // so that the down kernel's blocks read them from contiguous memory (in the [d_ff, ld] layout a row's n values are
    // followed by ld - n unused ones).
    const uint32_t act_ld = !z && p.n <= 2 && p.up_mode == HFFN_UP_EDGES && p.down_mode == HFFN_DOWN_EDGES ? p.n : p.ld;
    if (int status = launch_up(p.up_mode, p.value_type, x, p.up_offsets, p.up_idx, p.up_val, p.b_up, p.act, p.d_model, p.d_ff,
                               p.nnz_up, p.n, act_ld, s, z))
        return status;
    if (p.down_mode == HFFN_DOWN_ROWS)  // each output's lanes write y token-major: no output transpose
        return launched(hffn::launch_down_rows(p.value_type, p.act, p.out_offsets, p.out_hidden, p.out_val, p.b_down, p.y, p.d_model,
                                               p.n, p.ld, s, true),
                        "down rows");
    return launch_down(p.down_mode, p.value_type, p.act, p.out_offsets, p.out_hidden, p.out_val, p.b_down, p.y, p.d_model, p.d_ff,
                       p.nnz_down, p.n, act_ld, s);
}

// Everything of one decode-GEMV forward (hffn_forward_gemv) but x and the stream.
struct GemvPlan {
    int value_type;
    const void* up_planes;
    const int32_t* up_binades;
    const float* b_up;
    const void* down_planes;
    const int32_t* down_binades;
    const float* b_down;
    float* act;
    void* workspace;
    uint64_t workspace_bytes;
    float* y;
    uint32_t d_model, d_ff, n;
};

std::mutex g_plans_mutex;  // guards the plan tables and the handle counter (handles are unique across them)
std::unordered_map<uint64_t, Plan> g_plans;
std::unordered_map<uint64_t, GemvPlan> g_gemv_plans;
int check_tiles(int value_type, uint32_t d_model, uint32_t d_ff, uint32_t n) {
    if (!valid_value_type(value_type)) return fail(HFFN_ERROR_ARGUMENT, "unknown value type %d", value_type);
    if (d_model == 0 || d_model % 16 != 0 || d_model > HFFN_MAX_WIDTH || d_ff == 0 || d_ff % 8 != 0 || d_ff > HFFN_MAX_WIDTH)
        return fail(HFFN_ERROR_ARGUMENT, "tiles path: d_model=%u must be a multiple of 16 and d_ff=%u of 8, both at most %u", d_model,
                    d_ff, HFFN_MAX_WIDTH);
    if (n == 0 || n > hffn::kTilesMaxTokens) return fail(HFFN_ERROR_ARGUMENT, "tiles path: n=%u outside [1, %u]", n, hffn::kTilesMaxTokens);
    return HFFN_OK;
}

struct TilesPlan {
    int value_type;
    const void* up_store;  // the tiled stores; null for a plan on the compact rows
    const int32_t* up_table;
    const float* b_up;
    const void* down_store;
    const int32_t* down_table;
    const float* b_down;
    float* act;
    void* workspace;
    uint64_t workspace_bytes;
    float* y;
    uint32_t d_model, d_ff;
    uint64_t nnz_up, nnz_down;
    uint32_t n;
    const int16_t* up_idx = nullptr;  // the compact rows (hffn_forward_tiles_compact)
    const void* up_val = nullptr;
    const int16_t* out_hidden = nullptr;
    const void* out_val = nullptr;
};

int check_tiles_call(const TilesPlan& p, const float* x) {
    if (int status = check_tiles(p.value_type, p.d_model, p.d_ff, p.n)) return status;
    const bool compact = p.up_idx != nullptr;
    if (!x || !p.up_table || !p.b_up || !p.down_table || !p.b_down || !p.act || !p.workspace || !p.y ||
        (compact ? !p.up_val || !p.out_hidden || !p.out_val : !p.up_store || !p.down_store))
        return fail(HFFN_ERROR_ARGUMENT, "forward_tiles: null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(p.act) % 16 != 0)
        return fail(HFFN_ERROR_ARGUMENT, "forward_tiles: x and act must be 16-byte aligned");
    if (compact && (reinterpret_cast<uintptr_t>(p.up_idx) % 16 != 0 || reinterpret_cast<uintptr_t>(p.up_val) % 16 != 0 ||
                    reinterpret_cast<uintptr_t>(p.out_hidden) % 16 != 0 || reinterpret_cast<uintptr_t>(p.out_val) % 16 != 0))
        return fail(HFFN_ERROR_ARGUMENT, "forward_tiles_compact: the index and value arrays must be 16-byte aligned");
    if (!compact && (reinterpret_cast<uintptr_t>(p.up_store) % 16 != 0 || reinterpret_cast<uintptr_t>(p.down_store) % 16 != 0))
        return fail(HFFN_ERROR_ARGUMENT, "forward_tiles: the tiled stores must be 16-byte aligned");
    if (p.nnz_up > static_cast<uint64_t>(p.d_model) * p.d_ff || p.nnz_down > static_cast<uint64_t>(p.d_model) * p.d_ff)
        return fail(HFFN_ERROR_ARGUMENT, "forward_tiles: nnz_up=%llu / nnz_down=%llu beyond d_model * d_ff",
                    static_cast<unsigned long long>(p.nnz_up), static_cast<unsigned long long>(p.nnz_down));
    const uint64_t needed = hffn::tiles_workspace_bytes(p.value_type, p.n, p.d_model, p.d_ff, p.nnz_up, p.nnz_down);
    if (p.workspace_bytes < needed)
        return fail(HFFN_ERROR_ARGUMENT, "forward_tiles: workspace of %llu bytes, %llu needed for n=%u",
                    static_cast<unsigned long long>(p.workspace_bytes), static_cast<unsigned long long>(needed), p.n);
    return HFFN_OK;
}

int launch_tiles(const TilesPlan& p, const float* x, hipStream_t stream) {
    if (p.up_idx)
        return launched(hffn::launch_tiles_compact(p.value_type, x, p.up_idx, p.up_val, p.up_table, p.b_up, p.out_hidden, p.out_val,
                                                   p.down_table, p.b_down, p.act, static_cast<float*>(p.workspace), p.y, p.d_model,
                                                   p.d_ff, p.nnz_up, p.nnz_down, p.n, stream),
                        "forward (tiles, compact rows)");
    return launched(hffn::launch_tiles_forward(p.value_type, x, p.up_store, p.up_table, p.b_up, p.down_store, p.down_table, p.b_down,
                                               p.act, static_cast<float*>(p.workspace), p.y, p.d_model, p.d_ff, p.nnz_up, p.nnz_down,
                                               p.n, stream),
                    "forward (tiles)");
}

std::unordered_map<uint64_t, TilesPlan> g_tiles_plans;
uint64_t g_next_plan = 1;

}  // namespace

extern "C" {

int hffn_up(int mode, int value_type, const float* x, const int32_t* up_offsets, const int16_t* up_idx,
            const void* up_val, const float* b_up, float* act, uint32_t d_model, uint32_t d_ff, uint32_t nnz_up, uint32_t n,
            uint32_t ld, void* stream) {
    if (int status = check_up(mode, value_type, x, up_offsets, up_idx, up_val, b_up, act, d_model, d_ff, n, ld)) return status;
    return launch_up(mode, value_type, x, up_offsets, up_idx, up_val, b_up, act, d_model, d_ff, nnz_up, n, ld,
                     static_cast<hipStream_t>(stream));
}

int hffn_down(int mode, int value_type, const float* act, const int32_t* out_offsets, const int16_t* out_hidden,
              const void* out_val, const float* b_down, float* y, uint32_t d_model, uint32_t d_ff, uint32_t nnz_down,
              uint32_t n, uint32_t ld, void* stream) {
    if (int status = check_down(mode, value_type, act, out_offsets, out_hidden, out_val, b_down, y, d_model, d_ff, n, ld)) return status;
    return launch_down(mode, value_type, act, out_offsets, out_hidden, out_val, b_down, y, d_model, d_ff, nnz_down, n, ld,
                       static_cast<hipStream_t>(stream));
}

int hffn_forward(int up_mode, int down_mode, int value_type, const float* x, const int32_t* up_offsets,
                 const int16_t* up_idx, const void* up_val, const float* b_up, const int32_t* out_offsets,
                 const int16_t* out_hidden, const void* out_val, const float* b_down, float* x_t, float* act,
                 float* y_t, float* y, uint32_t d_model, uint32_t d_ff, uint32_t nnz_up, uint32_t nnz_down, uint32_t n,
                 uint32_t ld, void* stream) {
    const Plan plan{up_mode, down_mode, value_type, up_offsets, up_idx, up_val, b_up, out_offsets, out_hidden, out_val, b_down,
                    x_t, act, y_t, y, d_model, d_ff, nnz_up, nnz_down, n, ld};
    if (int status = check_forward(plan)) return status;
    if (!x) return fail(HFFN_ERROR_ARGUMENT, "forward: null input");
    return launch_forward(plan, x, static_cast<hipStream_t>(stream));
}

int hffn_plan_forward(int up_mode, int down_mode, int value_type, const int32_t* up_offsets, const int16_t* up_idx,
                      const void* up_val, const float* b_up, const int32_t* out_offsets, const int16_t* out_hidden,
                      const void* out_val, const float* b_down, float* x_t, float* act, float* y_t, float* y, uint32_t d_model,
                      uint32_t d_ff, uint32_t nnz_up, uint32_t nnz_down, uint32_t n, uint32_t ld, uint64_t* plan) {
    if (!plan) return fail(HFFN_ERROR_ARGUMENT, "plan_forward: null result");
    const Plan p{up_mode, down_mode, value_type, up_offsets, up_idx, up_val, b_up, out_offsets, out_hidden, out_val, b_down,
                 x_t, act, y_t, y, d_model, d_ff, nnz_up, nnz_down, n, ld};
    if (int status = check_forward(p)) return status;
    const std::lock_guard<std::mutex> lock(g_plans_mutex);
    *plan = g_next_plan++;
    g_plans.emplace(*plan, p);
    return HFFN_OK;
}

int hffn_plan_launch(uint64_t plan, const float* x, void* stream) {
    Plan p;
    GemvPlan g;
    TilesPlan t;
    bool gemv = false, tiles = false;
    {
        const std::lock_guard<std::mutex> lock(g_plans_mutex);
        if (const auto found = g_plans.find(plan); found != g_plans.end()) {
            p = found->second;
        } else if (const auto found_gemv = g_gemv_plans.find(plan); found_gemv != g_gemv_plans.end()) {
            g = found_gemv->second;
            gemv = true;
        } else if (const auto found_tiles = g_tiles_plans.find(plan); found_tiles != g_tiles_plans.end()) {
            t = found_tiles->second;
            tiles = true;
        } else {
            return fail(HFFN_ERROR_ARGUMENT, "plan_launch: unknown plan %llu", static_cast<unsigned long long>(plan));
        }
    }
    if (!x) return fail(HFFN_ERROR_ARGUMENT, "plan_launch: null input");
    if (tiles) {
        if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(HFFN_ERROR_ARGUMENT, "plan_launch: x must be 16-byte aligned");
        return launch_tiles(t, x, static_cast<hipStream_t>(stream));
    }
    if (gemv)  // the planned arguments passed their checks; x's alignment is checked here
        return hffn_forward_gemv(g.value_type, x, g.up_planes, g.up_binades, g.b_up, g.down_planes, g.down_binades, g.b_down, g.act,
                                 g.workspace, g.workspace_bytes, g.y, g.d_model, g.d_ff, g.n, stream);
    return launch_forward(p, x, static_cast<hipStream_t>(stream));
}

int hffn_plan_release(uint64_t plan) {
    const std::lock_guard<std::mutex> lock(g_plans_mutex);
    if (g_plans.erase(plan) == 0 && g_gemv_plans.erase(plan) == 0 && g_tiles_plans.erase(plan) == 0)
        return fail(HFFN_ERROR_ARGUMENT, "plan_release: unknown plan %llu", static_cast<unsigned long long>(plan));
    return HFFN_OK;
}

int hffn_output_major_workspace(uint32_t nnz, uint32_t d_model, uint64_t* bytes) {
    if (!bytes) return fail(HFFN_ERROR_ARGUMENT, "output_major_workspace: null result");
    *bytes = static_cast<uint64_t>(hffn::output_major_chunks(nnz)) * d_model * sizeof(int32_t);
    return HFFN_OK;
}

int hffn_output_major(int value_type, const int32_t* down_offsets, const int16_t* down_idx, const void* down_val,
                      uint32_t d_model, uint32_t d_ff, uint32_t nnz, int32_t* out_offsets, int16_t* out_hidden,
                      void* out_val, void* workspace, uint64_t workspace_bytes, void* stream) {
    if (!valid_value_type(value_type)) return fail(HFFN_ERROR_ARGUMENT, "unknown value type %d", value_type);
    if (d_model == 0 || d_model > HFFN_MAX_OUTPUT_MAJOR_WIDTH)
        return fail(HFFN_ERROR_ARGUMENT, "output_major: d_model=%u must be in [1, %u]", d_model, HFFN_MAX_OUTPUT_MAJOR_WIDTH);
    if (d_ff == 0 || d_ff > HFFN_MAX_WIDTH) return fail(HFFN_ERROR_ARGUMENT, "output_major: d_ff=%u must be in [1, %u]", d_ff, HFFN_MAX_WIDTH);
    if (!down_offsets || !out_offsets || !workspace || (nnz && (!down_idx || !down_val || !out_hidden || !out_val)))
        return fail(HFFN_ERROR_ARGUMENT, "output_major: null pointer");
    uint64_t needed = 0;
    hffn_output_major_workspace(nnz, d_model, &needed);
    if (workspace_bytes < needed)
        return fail(HFFN_ERROR_ARGUMENT, "output_major: workspace of %llu bytes, %llu needed", static_cast<unsigned long long>(workspace_bytes),
                    static_cast<unsigned long long>(needed));
    return launched(hffn::launch_output_major(value_type, down_offsets, down_idx, down_val, d_model, d_ff, nnz, out_offsets,
                                              out_hidden, out_val, static_cast<int32_t*>(workspace), static_cast<hipStream_t>(stream)),
                    "output_major");
}

int hffn_mfma_supported(uint32_t d_model, uint32_t d_ff) {
    return d_model <= HFFN_MAX_WIDTH && d_ff <= HFFN_MAX_WIDTH && hffn::mfma_shape_supported(d_model, d_ff) ? 1 : 0;
}

int hffn_dense_planes_bytes(uint32_t rows, uint32_t k, uint64_t* bytes) {
    if (!bytes) return fail(HFFN_ERROR_ARGUMENT, "dense_planes_bytes: null result");
    *bytes = static_cast<uint64_t>(hffn::dense_plane_halves(rows, k)) * 2;
    return HFFN_OK;
}

int hffn_densify(int value_type, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t k,
                 void* planes, int32_t* binades, void* stream) {
    if (!valid_value_type(value_type)) return fail(HFFN_ERROR_ARGUMENT, "unknown value type %d", value_type);
    if (rows == 0 || rows > HFFN_MAX_WIDTH || k == 0 || k % 32 != 0 || k > HFFN_MAX_WIDTH)
        return fail(HFFN_ERROR_ARGUMENT, "densify: rows=%u k=%u (k must be a positive multiple of 32)", rows, k);
    if (!offsets || !idx || !val || !planes || !binades) return fail(HFFN_ERROR_ARGUMENT, "densify: null pointer");
    return launched(hffn::launch_densify(value_type, offsets, idx, val, rows, k, planes, binades, static_cast<hipStream_t>(stream)),
                    "densify");
}

namespace {
int check_mfma(int value_type, uint32_t d_model, uint32_t d_ff, uint32_t n) {
    if (int status = check_shape(d_model, d_ff, n, (n + 3) / 4 * 4)) return status;
    if (!valid_value_type(value_type)) return fail(HFFN_ERROR_ARGUMENT, "unknown value type %d", value_type);
    if (!hffn_mfma_supported(d_model, d_ff))
        return fail(HFFN_ERROR_ARGUMENT, "mfma path: d_model=%u and d_ff=%u must be multiples of 256", d_model, d_ff);
    return HFFN_OK;
}
}  // namespace

int hffn_mfma_workspace(uint32_t n, uint32_t d_model, uint32_t d_ff, uint64_t* bytes) {
    if (!bytes) return fail(HFFN_ERROR_ARGUMENT, "mfma_workspace: null result");
    if (int status = check_mfma(HFFN_VALUE_F32, d_model, d_ff, n)) return status;
    *bytes = hffn::mfma_workspace_bytes(n, d_model, d_ff);
    return HFFN_OK;
}

int hffn_mfma_streamed(uint32_t n, uint32_t d_model, uint32_t d_ff) {
    if (int status = check_mfma(HFFN_VALUE_F32, d_model, d_ff, n)) return status;
    return hffn::mfma_streamed(n, d_model, d_ff) ? 1 : 0;
}

namespace {
int check_workspace(uint64_t bytes, uint32_t d_model, uint32_t d_ff, uint32_t n, const char* what) {
    const uint64_t needed = hffn::mfma_workspace_bytes(n, d_model, d_ff);
    if (bytes < needed)
        return fail(HFFN_ERROR_ARGUMENT, "%s: workspace of %llu bytes, %llu needed for n=%u", what, static_cast<unsigned long long>(bytes),
                    static_cast<unsigned long long>(needed), n);
    return HFFN_OK;
}
}  // namespace

int hffn_mfma_up(int value_type, const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up,
                 void* workspace, uint64_t workspace_bytes, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream) {
    if (int status = check_mfma(value_type, d_model, d_ff, n)) return status;
    if (!x || !up_planes || !up_binades || !b_up || !workspace) return fail(HFFN_ERROR_ARGUMENT, "mfma_up: null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(HFFN_ERROR_ARGUMENT, "mfma_up: x must be 16-byte aligned");
    if (int status = check_workspace(workspace_bytes, d_model, d_ff, n, "mfma_up")) return status;
    return launched(hffn::launch_mfma_up(value_type, x, up_planes, up_binades, b_up, workspace, n, d_model, d_ff,
                                         static_cast<hipStream_t>(stream)), "mfma up");
}

int hffn_mfma_split(const float* x, void* workspace, uint64_t workspace_bytes, uint32_t d_model, uint32_t d_ff, uint32_t n,
                    void* stream) {
    if (int status = check_mfma(HFFN_VALUE_F32, d_model, d_ff, n)) return status;
    if (!x || !workspace) return fail(HFFN_ERROR_ARGUMENT, "mfma_split: null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(HFFN_ERROR_ARGUMENT, "mfma_split: x must be 16-byte aligned");
    if (int status = check_workspace(workspace_bytes, d_model, d_ff, n, "mfma_split")) return status;
    return launched(hffn::launch_mfma_split(x, workspace, n, d_model, d_ff, static_cast<hipStream_t>(stream)), "mfma split");
}

int hffn_mfma_up_planes(int value_type, const void* up_planes, const int32_t* up_binades, const float* b_up, void* workspace,
                        uint64_t workspace_bytes, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream) {
    if (int status = check_mfma(value_type, d_model, d_ff, n)) return status;
    if (!up_planes || !up_binades || !b_up || !workspace) return fail(HFFN_ERROR_ARGUMENT, "mfma_up_planes: null pointer");
    if (int status = check_workspace(workspace_bytes, d_model, d_ff, n, "mfma_up_planes")) return status;
    return launched(hffn::launch_mfma_up_planes(value_type, up_planes, up_binades, b_up, workspace, n, d_model, d_ff,
                                                static_cast<hipStream_t>(stream)), "mfma up planes");
}

int hffn_mfma_down(int value_type, const void* down_planes, const int32_t* down_binades, const float* b_down, float* y,
                   void* workspace, uint64_t workspace_bytes, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream) {
    if (int status = check_mfma(value_type, d_model, d_ff, n)) return status;
    if (!down_planes || !down_binades || !b_down || !y || !workspace) return fail(HFFN_ERROR_ARGUMENT, "mfma_down: null pointer");
    if (int status = check_workspace(workspace_bytes, d_model, d_ff, n, "mfma_down")) return status;
    return launched(hffn::launch_mfma_down(value_type, down_planes, down_binades, b_down, y, workspace, n, d_model, d_ff,
                                           static_cast<hipStream_t>(stream)), "mfma down");
}

int hffn_forward_mfma(int value_type, const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up,
                      const void* down_planes, const int32_t* down_binades, const float* b_down, void* workspace,
                      uint64_t workspace_bytes, float* y, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream) {
    if (int status = hffn_mfma_up(value_type, x, up_planes, up_binades, b_up, workspace, workspace_bytes, d_model, d_ff, n, stream))
        return status;
    return hffn_mfma_down(value_type, down_planes, down_binades, b_down, y, workspace, workspace_bytes, d_model, d_ff, n, stream);
}

namespace {
int check_gemv(int value_type, uint32_t d_model, uint32_t d_ff, uint32_t n) {
    if (int status = check_mfma(value_type, d_model, d_ff, n)) return status;
    if (n > hffn::kGemvMaxTokens) return fail(HFFN_ERROR_ARGUMENT, "gemv path: n=%u above %u tokens", n, hffn::kGemvMaxTokens);
    return HFFN_OK;
}
}  // namespace

int hffn_gemv_workspace(uint32_t d_model, uint32_t d_ff, uint64_t* bytes) {
    if (!bytes) return fail(HFFN_ERROR_ARGUMENT, "gemv_workspace: null result");
    if (int status = check_gemv(HFFN_VALUE_F32, d_model, d_ff, 1)) return status;
    *bytes = hffn::gemv_workspace_bytes(d_model, d_ff);
    return HFFN_OK;
}

namespace {
int check_gemv_call(int value_type, const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up,
                    const void* down_planes, const int32_t* down_binades, const float* b_down, float* act, void* workspace,
                    uint64_t workspace_bytes, float* y, uint32_t d_model, uint32_t d_ff, uint32_t n) {
    if (int status = check_gemv(value_type, d_model, d_ff, n)) return status;
    if (!x || !up_planes || !up_binades || !b_up || !down_planes || !down_binades || !b_down || !act || !workspace || !y)
        return fail(HFFN_ERROR_ARGUMENT, "forward_gemv: null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(act) % 16 != 0)
        return fail(HFFN_ERROR_ARGUMENT, "forward_gemv: x and act must be 16-byte aligned");
    const uint64_t needed = hffn::gemv_workspace_bytes(d_model, d_ff);
    if (workspace_bytes < needed)
        return fail(HFFN_ERROR_ARGUMENT, "forward_gemv: workspace of %llu bytes, %llu needed",
                    static_cast<unsigned long long>(workspace_bytes), static_cast<unsigned long long>(needed));
    return HFFN_OK;
}
}  // namespace

int hffn_forward_gemv(int value_type, const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up,
                      const void* down_planes, const int32_t* down_binades, const float* b_down, float* act, void* workspace,
                      uint64_t workspace_bytes, float* y, uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream) {
    if (int status = check_gemv_call(value_type, x, up_planes, up_binades, b_up, down_planes, down_binades, b_down, act, workspace,
                                     workspace_bytes, y, d_model, d_ff, n))
        return status;
    return launched(hffn::launch_gemv_forward(value_type, x, up_planes, up_binades, b_up, down_planes, down_binades, b_down, act,
                                              static_cast<float*>(workspace), y, d_model, d_ff, n, static_cast<hipStream_t>(stream)),
                    "forward (gemv)");
}

int hffn_forward_gemv_static(int value_type, const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up,
                             const void* down_planes, const int32_t* down_binades, const float* b_down, float* act, float* y,
                             uint32_t d_model, uint32_t d_ff, uint32_t n, void* stream) {
    const uint64_t limit = hffn::gemv_scratch_bytes();
    if (int status = check_gemv(value_type, d_model, d_ff, n)) return status;
    const uint64_t needed = hffn::gemv_workspace_bytes(d_model, d_ff);
    if (needed > limit)
        return fail(HFFN_ERROR_ARGUMENT, "forward_gemv_static: d_model=%u d_ff=%u need %llu bytes of partials, beyond the %llu-byte static scratch",
                    d_model, d_ff, static_cast<unsigned long long>(needed), static_cast<unsigned long long>(limit));
    float* scratch = nullptr;
    if (int status = launched(hffn::gemv_scratch_address(&scratch), "forward_gemv_static: scratch address")) return status;
    if (int status = check_gemv_call(value_type, x, up_planes, up_binades, b_up, down_planes, down_binades, b_down, act, scratch,
                                     limit, y, d_model, d_ff, n))
        return status;
    return launched(hffn::launch_gemv_forward(value_type, x, up_planes, up_binades, b_up, down_planes, down_binades, b_down, act,
                                              scratch, y, d_model, d_ff, n, static_cast<hipStream_t>(stream)),
                    "forward (gemv, static scratch)");
}


int hffn_tiles_table_size(int value_type, uint32_t rows, uint32_t k, uint64_t* entries) {
    if (!entries) return fail(HFFN_ERROR_ARGUMENT, "tiles_table_size: null result");
    if (!valid_value_type(value_type)) return fail(HFFN_ERROR_ARGUMENT, "unknown value type %d", value_type);
    if (rows == 0 || rows > HFFN_MAX_WIDTH || k == 0 || k > HFFN_MAX_WIDTH)
        return fail(HFFN_ERROR_ARGUMENT, "tiles_table_size: rows=%u k=%u must be in [1, %u]", rows, k, HFFN_MAX_WIDTH);
    *entries = hffn::tiles_table_entries(value_type, rows, k);
    return HFFN_OK;
}

int hffn_tiles_table_build(int value_type, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t k,
                           int32_t* table, void* stream) {
    uint64_t entries = 0;
    if (int status = hffn_tiles_table_size(value_type, rows, k, &entries)) return status;
    if (!offsets || !idx || !val || !table) return fail(HFFN_ERROR_ARGUMENT, "tiles_table_build: null pointer");
    return launched(hffn::launch_tiles_table(value_type, offsets, idx, val, rows, k, table, static_cast<hipStream_t>(stream)),
                    "tiles table build");
}

int hffn_forward_tiles_compact(int value_type, const float* x, const int16_t* up_idx, const void* up_val, const int32_t* up_table,
                               const float* b_up, const int16_t* out_hidden, const void* out_val, const int32_t* down_table,
                               const float* b_down, float* act, void* workspace, uint64_t workspace_bytes, float* y, uint32_t d_model,
                               uint32_t d_ff, uint64_t nnz_up, uint64_t nnz_down, uint32_t n, void* stream) {
    TilesPlan p{value_type, nullptr, up_table, b_up, nullptr, down_table, b_down, act, workspace, workspace_bytes, y, d_model, d_ff, nnz_up,
                nnz_down, n, up_idx, up_val, out_hidden, out_val};
    if (!up_idx) return fail(HFFN_ERROR_ARGUMENT, "forward_tiles_compact: null pointer");
    if (int status = check_tiles_call(p, x)) return status;
    return launch_tiles(p, x, static_cast<hipStream_t>(stream));
}

int hffn_plan_tiles_compact(int value_type, const int16_t* up_idx, const void* up_val, const int32_t* up_table, const float* b_up,
                            const int16_t* out_hidden, const void* out_val, const int32_t* down_table, const float* b_down, float* act,
                            void* workspace, uint64_t workspace_bytes, float* y, uint32_t d_model, uint32_t d_ff, uint64_t nnz_up,
                            uint64_t nnz_down, uint32_t n, uint64_t* plan) {
    if (!plan) return fail(HFFN_ERROR_ARGUMENT, "plan_tiles_compact: null result");
    TilesPlan p{value_type, nullptr, up_table, b_up, nullptr, down_table, b_down, act, workspace, workspace_bytes, y, d_model, d_ff, nnz_up,
                nnz_down, n, up_idx, up_val, out_hidden, out_val};
    if (!up_idx) return fail(HFFN_ERROR_ARGUMENT, "plan_tiles_compact: null pointer");
    const float* some_x = reinterpret_cast<const float*>(uintptr_t{16});  // non-null, aligned: never dereferenced
    if (int status = check_tiles_call(p, some_x)) return status;
    const std::lock_guard<std::mutex> lock(g_plans_mutex);
    *plan = g_next_plan++;
    g_tiles_plans.emplace(*plan, p);
    return HFFN_OK;
}

int hffn_tiles_store_size(int value_type, uint32_t rows, uint32_t k, uint64_t nnz, uint64_t* store_bytes, uint64_t* table_entries) {
    if (!store_bytes || !table_entries) return fail(HFFN_ERROR_ARGUMENT, "tiles_store_size: null result");
    if (!valid_value_type(value_type)) return fail(HFFN_ERROR_ARGUMENT, "unknown value type %d", value_type);
    if (rows == 0 || rows > HFFN_MAX_WIDTH || k == 0 || k > HFFN_MAX_WIDTH)
        return fail(HFFN_ERROR_ARGUMENT, "tiles_store_size: rows=%u k=%u must be in [1, %u]", rows, k, HFFN_MAX_WIDTH);
    if (nnz > static_cast<uint64_t>(rows) * k)
        return fail(HFFN_ERROR_ARGUMENT, "tiles_store_size: nnz=%llu beyond rows * k", static_cast<unsigned long long>(nnz));
    const hffn::TilesStoreSize size = hffn::tiles_store_size(value_type, rows, k, nnz);
    *store_bytes = size.store_bytes;
    *table_entries = size.table_entries;
    return HFFN_OK;
}

int hffn_tiles_build(int value_type, const int32_t* offsets, const int16_t* idx, const void* val, uint32_t rows, uint32_t k,
                     uint64_t nnz, void* store, uint64_t store_bytes, int32_t* table, void* stream) {
    uint64_t needed = 0, entries = 0;
    if (int status = hffn_tiles_store_size(value_type, rows, k, nnz, &needed, &entries)) return status;
    if (!offsets || !idx || !val || !store || !table) return fail(HFFN_ERROR_ARGUMENT, "tiles_build: null pointer");
    if (reinterpret_cast<uintptr_t>(store) % 16 != 0) return fail(HFFN_ERROR_ARGUMENT, "tiles_build: the store must be 16-byte aligned");
    if (store_bytes < needed)
        return fail(HFFN_ERROR_ARGUMENT, "tiles_build: store of %llu bytes, %llu needed", static_cast<unsigned long long>(store_bytes),
                    static_cast<unsigned long long>(needed));
    return launched(hffn::launch_tiles_build(value_type, offsets, idx, val, rows, k, store, table, static_cast<hipStream_t>(stream)),
                    "tiles_build");
}

int hffn_tiles_workspace(int value_type, uint32_t n, uint32_t d_model, uint32_t d_ff, uint64_t nnz_up, uint64_t nnz_down,
                         uint64_t* bytes) {
    if (!bytes) return fail(HFFN_ERROR_ARGUMENT, "tiles_workspace: null result");
    if (int status = check_tiles(value_type, d_model, d_ff, n)) return status;
    if (nnz_up > static_cast<uint64_t>(d_model) * d_ff || nnz_down > static_cast<uint64_t>(d_model) * d_ff)
        return fail(HFFN_ERROR_ARGUMENT, "tiles_workspace: nnz_up=%llu / nnz_down=%llu beyond d_model * d_ff",
                    static_cast<unsigned long long>(nnz_up), static_cast<unsigned long long>(nnz_down));
    *bytes = hffn::tiles_workspace_bytes(value_type, n, d_model, d_ff, nnz_up, nnz_down);
    return HFFN_OK;
}

int hffn_forward_tiles(int value_type, const float* x, const void* up_store, const int32_t* up_table, const float* b_up,
                       const void* down_store, const int32_t* down_table, const float* b_down, float* act, void* workspace,
                       uint64_t workspace_bytes, float* y, uint32_t d_model, uint32_t d_ff, uint64_t nnz_up, uint64_t nnz_down,
                       uint32_t n, void* stream) {
    const TilesPlan p{value_type, up_store, up_table, b_up, down_store, down_table, b_down, act, workspace, workspace_bytes, y,
                      d_model, d_ff, nnz_up, nnz_down, n};
    if (int status = check_tiles_call(p, x)) return status;
    return launch_tiles(p, x, static_cast<hipStream_t>(stream));
}

int hffn_plan_tiles(int value_type, const void* up_store, const int32_t* up_table, const float* b_up, const void* down_store,
                    const int32_t* down_table, const float* b_down, float* act, void* workspace, uint64_t workspace_bytes, float* y,
                    uint32_t d_model, uint32_t d_ff, uint64_t nnz_up, uint64_t nnz_down, uint32_t n, uint64_t* plan) {
    if (!plan) return fail(HFFN_ERROR_ARGUMENT, "plan_tiles: null result");
    const TilesPlan p{value_type, up_store, up_table, b_up, down_store, down_table, b_down, act, workspace, workspace_bytes, y,
                      d_model, d_ff, nnz_up, nnz_down, n};
    const float* some_x = reinterpret_cast<const float*>(uintptr_t{16});  // non-null, aligned: never dereferenced
    if (int status = check_tiles_call(p, some_x)) return status;
    const std::lock_guard<std::mutex> lock(g_plans_mutex);
    *plan = g_next_plan++;
    g_tiles_plans.emplace(*plan, p);
    return HFFN_OK;
}

int hffn_plan_gemv(int value_type, const void* up_planes, const int32_t* up_binades, const float* b_up, const void* down_planes,
                   const int32_t* down_binades, const float* b_down, float* act, void* workspace, uint64_t workspace_bytes, float* y,
                   uint32_t d_model, uint32_t d_ff, uint32_t n, uint64_t* plan) {
    if (!plan) return fail(HFFN_ERROR_ARGUMENT, "plan_gemv: null result");
    const float* some_x = reinterpret_cast<const float*>(uintptr_t{16});  // non-null, aligned: never dereferenced
    if (int status = check_gemv_call(value_type, some_x, up_planes, up_binades, b_up, down_planes, down_binades, b_down, act, workspace,
                                     workspace_bytes, y, d_model, d_ff, n))
        return status;
    const GemvPlan g{value_type, up_planes, up_binades, b_up, down_planes, down_binades, b_down, act, workspace, workspace_bytes,
                     y, d_model, d_ff, n};
    const std::lock_guard<std::mutex> lock(g_plans_mutex);
    *plan = g_next_plan++;
    g_gemv_plans.emplace(*plan, g);
    return HFFN_OK;
}

// ----------------------------------------------------------------------------------------------------- training

int hffn_forward_z(int up_mode, int down_mode, const float* x, const int32_t* up_offsets, const int16_t* up_idx, const float* up_val,
                   const float* b_up, const int32_t* out_offsets, const int16_t* out_hidden, const float* out_val, const float* b_down,
                   float* x_t, float* act, float* y_t, float* y, float* z, uint32_t d_model, uint32_t d_ff, uint32_t nnz_up,
                   uint32_t nnz_down, uint32_t n, uint32_t ld, void* stream) {
    const Plan plan{up_mode, down_mode, HFFN_VALUE_F32, up_offsets, up_idx, up_val, b_up, out_offsets, out_hidden, out_val, b_down,
                    x_t, act, y_t, y, d_model, d_ff, nnz_up, nnz_down, n, ld};
    if (int status = check_forward(plan)) return status;
    if (!x || !x_t || !z) return fail(HFFN_ERROR_ARGUMENT, "forward_z: null input, x_t or z");
    return launch_forward(plan, x, static_cast<hipStream_t>(stream), z);
}

int hffn_grad_dense_workspace(uint32_t rows, uint32_t cols, uint32_t n, uint64_t* bytes) {
    if (!bytes) return fail(HFFN_ERROR_ARGUMENT, "grad_dense_workspace: null result");
    if (int status = check_shape(16, rows, n, (n + 3) / 4 * 4)) return status;
    if (cols == 0 || cols > HFFN_MAX_WIDTH) return fail(HFFN_ERROR_ARGUMENT, "grad_dense: cols=%u", cols);
    const size_t needed = hffn::grad_dense_workspace_bytes(rows, cols, n);
    if (needed == 0)
        return fail(HFFN_ERROR_ARGUMENT, "grad_dense: rows=%u cols=%u n=%u do not run on the streamed GEMM (multiples of 256, enough tiles)",
                    rows, cols, n);
    *bytes = needed;
    return HFFN_OK;
}

int hffn_grad_dense(const float* row, const float* mat, const int32_t* offsets, const int16_t* index, float* g, float* gb,
                    uint32_t rows, uint32_t cols, uint32_t n, uint32_t ld, void* workspace, uint64_t workspace_bytes, void* stream) {
    uint64_t needed = 0;
    if (int status = hffn_grad_dense_workspace(rows, cols, n, &needed)) return status;
    if (ld < n || ld % 4 != 0) return fail(HFFN_ERROR_ARGUMENT, "grad_dense: ld=%u must be a multiple of 4 and at least n=%u", ld, n);
    if (!row || !mat || !offsets || !index || !g || !gb || !workspace) return fail(HFFN_ERROR_ARGUMENT, "grad_dense: null pointer");
    if (reinterpret_cast<uintptr_t>(row) % 16 != 0 || reinterpret_cast<uintptr_t>(mat) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return fail(HFFN_ERROR_ARGUMENT, "grad_dense: row and mat must be 16-byte aligned, the workspace 256-byte aligned");
    if (workspace_bytes < needed)
        return fail(HFFN_ERROR_ARGUMENT, "grad_dense: workspace of %llu bytes, %llu needed", static_cast<unsigned long long>(workspace_bytes),
                    static_cast<unsigned long long>(needed));
    return launched(hffn::launch_grad_dense(row, mat, offsets, index, g, gb, rows, cols, n, ld, workspace, static_cast<hipStream_t>(stream)),
                    "grad_dense");
}

int hffn_train_mfma_workspace(uint32_t n, uint32_t d_model, uint32_t d_ff, uint64_t* bytes) {
    if (!bytes) return fail(HFFN_ERROR_ARGUMENT, "train_mfma_workspace: null result");
    if (int status = check_mfma(HFFN_VALUE_F32, d_model, d_ff, n)) return status;
    if (!hffn::mfma_streamed(n, d_model, d_ff))
        return fail(HFFN_ERROR_ARGUMENT, "train_mfma: the streamed GEMM does not take n=%u on %u x %u", n, d_model, d_ff);
    *bytes = hffn::train_mfma_workspace_bytes(n, d_model, d_ff);
    return HFFN_OK;
}

namespace {
int check_train_mfma(const char* what, uint32_t d_model, uint32_t d_ff, uint32_t n, uint32_t ld, const void* workspace,
                     uint64_t workspace_bytes, std::initializer_list<const void*> floats, std::initializer_list<const void*> others) {
    uint64_t needed = 0;
    if (int status = hffn_train_mfma_workspace(n, d_model, d_ff, &needed)) return status;
    if (ld < n || ld % 4 != 0) return fail(HFFN_ERROR_ARGUMENT, "%s: ld=%u must be a multiple of 4 and at least n=%u", what, ld, n);
    for (const void* p : floats)
        if (!p || reinterpret_cast<uintptr_t>(p) % 16 != 0) return fail(HFFN_ERROR_ARGUMENT, "%s: null or not 16-byte aligned float buffer", what);
    for (const void* p : others)
        if (!p) return fail(HFFN_ERROR_ARGUMENT, "%s: null pointer", what);
    if (!workspace || reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return fail(HFFN_ERROR_ARGUMENT, "%s: the workspace must be 256-byte aligned", what);
    if (workspace_bytes < needed)
        return fail(HFFN_ERROR_ARGUMENT, "%s: workspace of %llu bytes, %llu needed", what, static_cast<unsigned long long>(workspace_bytes),
                    static_cast<unsigned long long>(needed));
    return HFFN_OK;
}
}  // namespace

int hffn_forward_mfma_z(const float* x, const void* up_planes, const int32_t* up_binades, const float* b_up, const void* down_planes,
                        const int32_t* down_binades, const float* b_down, void* workspace, uint64_t workspace_bytes, float* x_t,
                        float* act, float* z, float* y, uint32_t d_model, uint32_t d_ff, uint32_t n, uint32_t ld, void* stream) {
    if (int status = check_train_mfma("forward_mfma_z", d_model, d_ff, n, ld, workspace, workspace_bytes,
                                      {x, b_up, b_down, x_t, act, z, y, up_planes, down_planes}, {up_binades, down_binades}))
        return status;
    return launched(hffn::launch_train_forward(x, up_planes, up_binades, b_up, down_planes, down_binades, b_down, workspace, x_t, act, z, y,
                                               n, d_model, d_ff, ld, static_cast<hipStream_t>(stream)),
                    "forward_mfma_z");
}

int hffn_backward_mfma(const float* gy, const float* z, const void* down_t_planes, const int32_t* down_t_binades, const void* up_t_planes,
                       const int32_t* up_t_binades, void* workspace, uint64_t workspace_bytes, float* gz, float* gx, uint32_t d_model,
                       uint32_t d_ff, uint32_t n, uint32_t ld, void* stream) {
    if (int status = check_train_mfma("backward_mfma", d_model, d_ff, n, ld, workspace, workspace_bytes,
                                      {gy, z, gz, gx, down_t_planes, up_t_planes}, {down_t_binades, up_t_binades}))
        return status;
    return launched(hffn::launch_train_backward(gy, z, down_t_planes, down_t_binades, up_t_planes, up_t_binades, workspace, gz, gx, n,
                                                d_model, d_ff, ld, static_cast<hipStream_t>(stream)),
                    "backward_mfma");
}

int hffn_grad_sddmm(const float* row, const float* mat, const int32_t* offsets, const int16_t* index, float* g, float* gb,
                    uint32_t rows, uint32_t n, uint32_t ld, uint32_t stride, void* stream) {
    if (int status = check_shape(16, rows, n, ld)) return status;
    if (!row || !mat || !offsets || !index || !g || !gb) return fail(HFFN_ERROR_ARGUMENT, "grad_sddmm: null pointer");
    if (reinterpret_cast<uintptr_t>(row) % 16 != 0 || reinterpret_cast<uintptr_t>(mat) % 16 != 0)
        return fail(HFFN_ERROR_ARGUMENT, "grad_sddmm: row and mat must be 16-byte aligned");
    if (hffn::grad_tiles(n) > 1 && stride == 0) return fail(HFFN_ERROR_ARGUMENT, "grad_sddmm: n=%u needs a partial stride", n);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (n <= hffn::kEdgesMaxTokens) {
        if (ld % hffn::edges_tokens(n) != 0) return fail(HFFN_ERROR_ARGUMENT, "grad_sddmm: ld=%u must be a multiple of %u", ld, hffn::edges_tokens(n));
        return launched(hffn::launch_grad_sddmm_edges(row, mat, offsets, index, g, gb, rows, n, ld, s), "grad_sddmm (edges)");
    }
    return launched(hffn::launch_grad_sddmm(row, mat, offsets, index, g, gb, rows, n, ld, stride, s), "grad_sddmm");
}

int hffn_grad_hidden(const float* gy, const float* gy_t, const float* z, const int32_t* down_offsets, const int16_t* down_idx,
                     const float* down_val, float* gz, uint32_t d_model, uint32_t d_ff, uint32_t nnz_down, uint32_t n, uint32_t ld,
                     void* stream) {
    if (int status = check_shape(d_model, d_ff, n, ld)) return status;
    if (!gy || !gy_t || !z || !down_offsets || !down_idx || !down_val || !gz) return fail(HFFN_ERROR_ARGUMENT, "grad_hidden: null pointer");
    if (reinterpret_cast<uintptr_t>(gy_t) % 16 != 0) return fail(HFFN_ERROR_ARGUMENT, "grad_hidden: gy_t must be 16-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (n <= hffn::kEdgesMaxTokens && hffn_edges_supported(d_model, n) && check_edges(d_model, n, ld, true) == HFFN_OK) {
        if (int status = check_store_alignment(down_idx, down_val, HFFN_VALUE_F32)) return status;
        return launched(hffn::launch_grad_hidden_edges(gy, down_offsets, down_idx, down_val, z, gz, d_model, d_ff, n, ld, nnz_down, s),
                        "grad_hidden (edges)");
    }
    return launched(hffn::launch_grad_hidden_rows(gy_t, down_offsets, down_idx, down_val, z, gz, d_ff, n, ld, s), "grad_hidden");
}

int hffn_grad_x(const float* gz, const int32_t* in_offsets, const int16_t* in_hidden, const float* in_val, float* gx_t, float* gx,
                uint32_t d_model, uint32_t d_ff, uint32_t nnz_up, uint32_t n, uint32_t ld, void* stream) {
    if (int status = check_shape(d_model, d_ff, n, ld)) return status;
    if (!gz || !in_offsets || !in_hidden || !in_val || !gx_t || !gx) return fail(HFFN_ERROR_ARGUMENT, "grad_x: null pointer");
    if (reinterpret_cast<uintptr_t>(gz) % 16 != 0) return fail(HFFN_ERROR_ARGUMENT, "grad_x: gz must be 16-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (n <= hffn::kEdgesMaxTokens && check_edges(d_model, n, ld, false) == HFFN_OK) {
        if (int status = check_store_alignment(in_hidden, in_val, HFFN_VALUE_F32)) return status;
        return launched(hffn::launch_down_edges(HFFN_VALUE_F32, gz, in_offsets, in_hidden, in_val, nullptr, gx, d_model, d_ff, n, ld,
                                                nnz_up, s),
                        "grad_x (edges)");
    }
    if (int status = launched(hffn::launch_down_rows(HFFN_VALUE_F32, gz, in_offsets, in_hidden, in_val, nullptr, gx_t, d_model, n,
                                                     ld, s),
                              "grad_x"))
        return status;
    return launched(hffn::launch_transpose(gx_t, gx, d_model, n, ld, d_model, s), "grad_x transpose");
}

int hffn_reduce_tiles(const float* ws, uint32_t stride, uint32_t tiles, uint32_t c1, uint32_t c2, uint32_t c3, float* g_down,
                      float* gb_down, float* g_up, float* gb_up, void* stream) {
    if (!ws || !g_down || !gb_down || !g_up || !gb_up) return fail(HFFN_ERROR_ARGUMENT, "reduce_tiles: null pointer");
    if (tiles == 0 || !(c1 <= c2 && c2 <= c3 && c3 <= stride))
        return fail(HFFN_ERROR_ARGUMENT, "reduce_tiles: columns %u <= %u <= %u <= %u and tiles=%u >= 1 required", c1, c2, c3, stride, tiles);
    if (static_cast<uint64_t>(tiles) * stride >= (1ull << 32)) return fail(HFFN_ERROR_ARGUMENT, "reduce_tiles: workspace beyond 32-bit indexing");
    return launched(hffn::launch_reduce_tiles(ws, stride, tiles, c1, c2, c3, g_down, gb_down, g_up, gb_up, static_cast<hipStream_t>(stream)),
                    "reduce_tiles");
}

int hffn_adamw(float* p, const float* g, float* m, float* v, uint32_t count, float lr_decay, float beta1, float one_minus_beta1,
               float beta2, float one_minus_beta2, float step_size, float bias2_sqrt, float eps, void* stream) {
    if (count == 0) return HFFN_OK;
    if (!p || !g || !m || !v) return fail(HFFN_ERROR_ARGUMENT, "adamw: null pointer");
    return launched(hffn::launch_adamw(p, g, m, v, count, lr_decay, beta1, one_minus_beta1, beta2, one_minus_beta2, step_size, bias2_sqrt,
                                       eps, static_cast<hipStream_t>(stream)),
                    "adamw");
}

int hffn_gather_values(const float* src, const int32_t* pos, float* dst, uint32_t count, void* stream) {
    if (count == 0) return HFFN_OK;
    if (!src || !pos || !dst) return fail(HFFN_ERROR_ARGUMENT, "gather_values: null pointer");
    return launched(hffn::launch_gather_values(src, pos, dst, count, static_cast<hipStream_t>(stream)), "gather_values");
}

int hffn_read_probe(const void* data, uint64_t bytes, uint32_t* sink, uint32_t sink_words, uint32_t blocks, void* stream) {
    if (!data || !sink) return fail(HFFN_ERROR_ARGUMENT, "read_probe: null pointer");
    if (bytes == 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(data) % 16 != 0)
        return fail(HFFN_ERROR_ARGUMENT, "read_probe: %llu bytes: a nonzero multiple of 16 bytes from a 16-byte aligned pointer",
                    static_cast<unsigned long long>(bytes));
    if (blocks == 0 || blocks > 65535 || static_cast<uint64_t>(sink_words) < 4ull * blocks)
        return fail(HFFN_ERROR_ARGUMENT, "read_probe: %u blocks need 1-65535 blocks and 4 sink words each (%u given)", blocks, sink_words);
    return launched(hffn::launch_read_probe(data, bytes, sink, blocks, static_cast<hipStream_t>(stream)), "read_probe");
}

}  // extern "C"
