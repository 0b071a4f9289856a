// hf_api_internal.h -- library state shared by the C-ABI translation units.
#pragma once

#include <algorithm>
#include <cstdint>
#include <map>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "expert_stream_policy.h"
#include "hfmoe.h"
#include "hf_kernels.h"

namespace hf {

struct Workspace {
    float* logits = nullptr;     // [maxT, E]
    float2* scores = nullptr;    // [maxT, E] (sigmoid, sigmoid + bias)
    int* idx = nullptr;          // [maxT, k]
    float* wts = nullptr;        // [maxT, k]
    float* h = nullptr;          // [k + n_shared, I]  (T = 1 path)
    unsigned int* counter = nullptr;
    float* x_io = nullptr;       // [d]  host-contract staging
    float* out_io = nullptr;     // [d]
    float* io_pin = nullptr;     // pinned host [2, d], coherent: the host contract's x, then out
    float* io_pin_dev = nullptr; // its device address (null: copies go through hipMemcpyAsync)
    float* tmp = nullptr;        // [2, maxT, d] (mlp block: normed x, MoE out; BF16 x widened)
};

// Buffers of the multi-token (dispatch + grouped) path.  Sorted rows: the
// maxT*k routed (token, rank) pairs by expert, then maxT shared-expert rows.
struct GroupedWorkspace {
    int* counts = nullptr;       // [E]
    int* offsets = nullptr;      // [E + 2] group row offsets (group E = shared expert)
    int* perm = nullptr;         // [rows] pair id (y row) of each sorted row
    int* row_token = nullptr;    // [rows] token of each sorted row
    int* tile_expert = nullptr;  // [max_tiles] group of each M tile
    int* tile_row0 = nullptr;    // [max_tiles] first sorted row of each M tile
    int* ntiles = nullptr;       // [64] M tiles in use: [0] this list, [kWideCountAt] the wide list
    static constexpr int kWideCountAt = 32;  // its own 128-byte line
    int* ntiles_wide() const { return ntiles + kWideCountAt; }
    int* tile_expert_gu = nullptr;  // [max_tiles] the wide kernel's tiles (kWideTileRows rows)
    int* tile_row0_gu = nullptr;
    bool wide = false;              // the last dispatch wrote that list (the GEMMs after it take the wide tiles)
    int* chunk_hist = nullptr;   // [kDispatchMaxChunks, E] dispatch chunk counts / first slots
    unsigned* item_ctr = nullptr;  // [kItemCounters] prefill GEMM work counters (zeroed by the dispatch)
    unsigned int* lo_flag = nullptr;  // [0] x has a nonzero BF16 lo half
    uint16_t* xh = nullptr;      // [maxT, d] x BF16 hi (token order)
    uint16_t* xl = nullptr;      // [maxT, d] x BF16 lo
    uint16_t* hh = nullptr;      // [rows, I] h hi (sorted rows)
    uint16_t* hl = nullptr;      // [rows, I] h lo
    float* y = nullptr;          // [rows, d] expert outputs at pair slots, shared rows after
    float* part = nullptr;       // [ksplit, maxT, E] router split-K partials
    int max_tiles = 0;
};

struct LayerState {
    int location = HFMOE_EXPERTS_DEVICE;
    LayerDev dev{};
    const uint16_t** etab_dev = nullptr;
    std::vector<const uint16_t*> host_experts;  // 3*E as registered
    const uint16_t* norm_w = nullptr;
    // Dense MLP layer: dev.sg / su / sd hold its gate, up and down matrices
    // ([inter, d], [inter, d], [d, inter]), multiplied as dense_inter / dense_slice
    // slices of dense_slice rows by the decode kernels.
    bool dense = false;
    int dense_inter = 0;
    int dense_slice = 0;
};

// The LM head (lm_head.hip): caller-owned weights, the library's partial
// argmax buffer.
struct LmHead {
    const uint16_t* w = nullptr;     // [vocab, d]
    const uint16_t* norm = nullptr;  // final RMSNorm weight [d] or null
    int vocab = 0;
    void* part = nullptr;            // per-block winners of the T = 1 GEMV
    int part_n = 0;                  // their number: the most workgroups that GEMV takes
};

// Buffers of the dense-MLP layers (sized for the largest registered inter).
struct DenseWorkspace {
    float* h1 = nullptr;     // [inter] T = 1 intermediate
    uint16_t* hh = nullptr;  // [max_tokens, inter] h hi (multi-token path)
    uint16_t* hl = nullptr;  // [max_tokens, inter] h lo
    float* part = nullptr;   // [part_rows, hidden] K-split partials of the down projection
    float* gu_part = nullptr;  // [gu_part_rows, 2 inter] K-split gate / up partials
    int inter = 0;
    int tokens = 0;
    int part_rows = 0;       // max(2 * max_tokens, min(8 * max_tokens, 4096))
    int gu_part_rows = 0;    // splits x tokens the gate/up partials hold
};

struct Pending {
    const char* name = nullptr;
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

// Staging pool of the streamed-expert path: HBM slots that receive selected
// (and predicted) experts from pinned host RAM on the copy stream.  Which
// slot holds what is decided by `policy`.
struct StreamPool {
    int slots = 0;
    size_t slot_bytes = 0;
    uint16_t* base = nullptr;
    std::vector<hipEvent_t> copied;   // per slot: H2D done (copy stream)
    std::vector<hipEvent_t> consumed; // per slot: last kernel reading it done
    ExpertStreamPolicy policy;
    // Small transfers between the compute stream and the host go through
    // mapped pinned memory, read or written by a kernel on that stream: a DMA
    // copy there could queue behind expert weight copies.
    int* idx_host = nullptr;          // pinned, mapped [k] selected experts readback
    float* w_host = nullptr;          // pinned, mapped [k] their routing weights
    const uint16_t** etab_host = nullptr;  // pinned, mapped [3*k] slot pointers for the table
    int* idx_host_dev = nullptr;      // device addresses of the three
    float* w_host_dev = nullptr;
    const uint16_t** etab_host_dev = nullptr;
    const uint16_t** etab_dev = nullptr;   // device [3*k] slot pointers of this call
    int* iota_dev = nullptr;               // device [k] = 0..k-1 (slot order)
    float* shared_out = nullptr;           // device [d] shared-expert output
    hipEvent_t routed = nullptr;
    // Multi-token calls: the batch's selections read back, and one pinned
    // staging table of 3 * (E + 1) slot pointers per wave of experts (a wave's
    // table is copied to the layer's device table while the host fills the next).
    int* idx_batch_host = nullptr;         // pinned, mapped [max_tokens * k]
    float* w_batch_host = nullptr;         // pinned, mapped [max_tokens * k] routing weights
    int* idx_batch_host_dev = nullptr;
    float* w_batch_host_dev = nullptr;
    const uint16_t** wave_tabs = nullptr;  // pinned, mapped [max_waves][3 * (E + 1)]
    const uint16_t** wave_tabs_dev = nullptr;  // its device address (a kernel copies a table in)
    int max_waves = 0;
};

struct State {
    bool inited = false;
    bool configured = false;
    int device = -1;
    int num_cus = 0;
    size_t total_mem = 0;
    char name[256] = {0};
    hipStream_t stream = nullptr;
    hipStream_t copy_stream = nullptr;
    Cfg cfg{};
    int max_tokens = 1;
    uint64_t vram_budget = 0;
    std::map<int, LayerState> layers;
    Workspace ws;
    GroupedWorkspace gws;
    DenseWorkspace dws;
    LmHead lm;
    StreamPool pool;
    StreamPolicyOptions stream_opt;   // kept across hfmoe_configure
    // profiling / telemetry
    bool prof_on = false;
    std::vector<Pending> pending;
    std::vector<hipEvent_t> event_pool;
    std::map<std::string, std::pair<int64_t, double>> kstats;
    uint64_t pcie_bytes = 0;
    uint64_t gpu_active_ns = 0;
    std::string last_error;
};

extern State g;

int fail(int code, const char* fmt, ...);
int fail_hip(hipError_t e, const char* what);
int require_init();
int require_cfg();
int env_int(const char* name, int dflt);
// HFMOE_ERR_INVALID_ARGUMENT naming the layer and tensor when p % align != 0.
int check_align(int layer, const char* what, const void* p, size_t align);
hipStream_t pick_stream(void* s);
void prof_begin(Pending& p, const char* name, hipStream_t s);
void prof_end(Pending& p, hipStream_t s);
void prof_drain();

// Scratch of the T = 1 decode kernels: router logits [E], score pairs [E],
// selected ids [k], routing weights [k], h [k + n_shared, I].
struct T1Buffers {
    float* logits;
    float2* scores;
    int* idx;
    float* wts;
    float* h;
};

// forward.hip
int gu_blocks();
int dn_blocks();
int forward_t1(LayerState& L, const float* x, float* out, hipStream_t s, const hfmoe_route_debug* dbg);
// The decode launches over explicit scratch; profile = false records no timing
// events (so the call creates none).
int forward_t1_on(LayerState& L, const float* x, float* out, hipStream_t s, const T1Buffers& b, bool profile);
// noalloc.hip: the device address of this device's static scratch array
// (hipGetSymbolAddress, once per device; called by hfmoe_init).
void noalloc_setup(int device);  // never fails init: see noalloc.hip
int forward_tokenwise(LayerState& L, const float* x, int T, float* out, hipStream_t s,
                      const hfmoe_route_debug* dbg);
int copy_debug(const hfmoe_route_debug* dbg, int T, hipStream_t s);
// grouped_forward.hip
int forward_grouped(LayerState& L, const float* x, int T, float* out, hipStream_t s,
                    const hfmoe_route_debug* dbg);
// The three phases of forward_grouped (multi-token path, grouped workspace
// allocated): routing (x split, router, selection, dispatch), the expert
// gate/up and down GEMMs of the groups whose etab entries are not null (3 per
// group, E + 1 groups, the shared expert last), and the weighted combine.
int grouped_route(LayerState& L, const float* x, int T, hipStream_t s);
int grouped_experts(const uint16_t* const* etab, int T, hipStream_t s);
int grouped_combine(int T, float* out, hipStream_t s);
int grouped_tile_rows(int T);
int grouped_workspace_alloc();
void grouped_workspace_free();
int gemm_blocks(int tile_rows);
// dense.hip
int dense_forward(LayerState& L, const float* x, int T, float* out, hipStream_t s);
void dense_workspace_free();
// lm_head.hip
void lm_head_release();
hipError_t launch_row_argmax(const float* x, int T, int n, int* out, hipStream_t s);
hipError_t launch_matvec_bf16(const uint16_t* W, const float* x, int M, int K, float* y, hipStream_t s);
// streamed.hip
int streamed_forward_t1(int layer, LayerState& L, const float* x, float* out, hipStream_t s,
                        const hfmoe_route_debug* dbg);
// T > 1 over the grouped GEMMs: the batch's distinct experts in waves that fit
// the slot pool (grouped workspace required).
int streamed_forward_batch(int layer, LayerState& L, const float* x, int T, float* out, hipStream_t s,
                           const hfmoe_route_debug* dbg);
void stream_pool_release();
// misc kernels
hipError_t launch_rmsnorm(const float* h, const uint16_t* w, float* out, int T, int d, float eps,
                          hipStream_t s);
hipError_t launch_add_inplace(float* dst, const float* src, size_t n, hipStream_t s);
hipError_t launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t s);
hipError_t launch_bf16_to_f32(const uint16_t* src, float* dst, size_t n, hipStream_t s);
// dst[0, n) = src[0, n) by a kernel (either may be mapped pinned host memory).
hipError_t launch_copy_u32(const uint32_t* src, uint32_t* dst, size_t n, hipStream_t s);
hipError_t launch_copy_u64(const uint64_t* src, uint64_t* dst, size_t n, hipStream_t s);

}  // namespace hf
