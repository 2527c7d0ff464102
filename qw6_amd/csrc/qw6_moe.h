// qw6_moe.h -- types shared by the decode (qw6_hip.hip) and batched
// (qw6_prefill.hip) MoE FFN paths, and the batched path's host entry.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qw6 {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// A load through a pointer to device global memory, emitted as a global
// load. A load through a generic pointer whose address space the compiler
// cannot infer (one read from memory, or a select of such pointers) is a
// FLAT load, which also counts in lgkmcnt: every later wait for an LDS
// operation then waits for it too, and a load issued ahead for the next
// step holds up the current step's LDS reads.
template <typename T>
__device__ __forceinline__ T ld_global(const void* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}

// One weight matrix on the device (fmt: internal format, -1 = F32).
struct MatD {
    const uint8_t* p;
    int32_t fmt;
    uint32_t rows, cols, rb;   // rb: bytes per row
};

struct ExpertEnt {            // device expert table entry
    const uint8_t* p[3];      // gate, up, down
    int32_t fmt[3];
    uint32_t rb[3];
};

// Addressing of one matrix kind (gate / up / down) of the experts: a regular
// pack (expert e at base + e * stride, one format; the GGUF expert pack of
// bind_expert_pack, qw6.c:542-597) needs no memory round trip; otherwise the
// per-expert table entry is loaded.
struct PackRef {
    const uint8_t* base;
    uint64_t stride;
    int32_t fmt;
    uint32_t rb;
    uint32_t regular;
};

// Device workspace of the batched path, sized for max_tokens tokens.
struct PrefillWs {
    uint32_t* pidx;      // [T][top_k] selected experts
    float* pw;           // [T][top_k] gate weights
    uint32_t* ent_tok;   // [E] token of each entry (entries grouped by expert)
    float* ent_w;        // [E] gate weight of each entry
    uint32_t* ent_pos;   // [T][top_k] entry of (token, k)
    uint4* tiles;        // [n_tiles_max] {matrix id, first entry, count, 0}
    uint32_t* n_tiles;   // [2] routed tiles, shared tiles
    uint32_t* forder;    // [2][n_tiles_max] tile indices grouped by format (gate/up, down)
    uint32_t* fseg;      // [2][8][2] {first, count} of each format's group in forder
    float* logits;       // [T][n_experts]
    float* xn;           // [T][hidden] (RMSNorm of the input)
    uint16_t* xp[3];     // [T][hidden] each: the input's P bf16 parts, part p at xp[p]
                         // (hi, then lo for P = 2; hi, mid, lo for P = 3)
    uint16_t* mp[3];     // [E][inter] each: the same parts of silu(gate) * up
    uint16_t* xs3;       // [T][hidden / 256][3][8] input sums per 32 columns, 3 bf16 parts
    uint16_t* ms3;       // [E][inter / 256][3][8] the same for mid
    float* ybuf;         // [E][hidden]
};

struct PrefillLayer {
    uint32_t hidden, inter, n_experts, top_k, T;
    const float* x;
    const float* logits;          // given router logits or nullptr
    const float* router;          // F32 router or nullptr
    const float* shared_router;   // nullptr: shared weight 1
    const float* norm_w;          // RMSNorm weight or nullptr
    float norm_eps;
    const float* residual;
    float* out;
    uint32_t* idx_out;
    float* w_out;
    const ExpertEnt* experts;
    PackRef pk[3];
    uint32_t fmask_gu, fmask_dn;  // formats of the routed experts' gate/up (down): bit f
    MatD sg, su, sd;              // shared expert (sg.p == nullptr: none)
};

// Entries of a batch of T tokens: T * top_k routed, then T shared.
inline uint32_t prefill_entries(uint32_t T, uint32_t top_k) { return T * top_k + T; }
// Entries per tile of the grouped kernels (one MFMA row group).
constexpr uint32_t kPrefillTileEntries = 16;
// Calls of fewer tokens split the activations into three bf16 parts (hi,
// mid, lo: 24 significant bits, the fp32 bar); from this many on into two
// (hi, lo: 16 bits), the bf16-MFMA bar, at the lower LDS cost.
constexpr uint32_t kPrefill3PartBelow = 64;
// Tiles of a batch at most: the routed entries in tiles of one expert each
// (at most one partial tile per expert), then the shared expert's.
__host__ __device__ inline uint32_t prefill_tiles_max(uint32_t T, uint32_t top_k, uint32_t n_experts) {
    const uint32_t m = kPrefillTileEntries;
    return (T * top_k + m - 1) / m + n_experts + (T + m - 1) / m;
}
// Formats the grouped kernels decode (others take the per-token kernels).
bool prefill_supports(int fmt);
// Launch the batched MoE FFN on `st`; 0 or -1 (message via qw6_fail).
int prefill_forward(const PrefillLayer& L, const PrefillWs& ws, hipStream_t st);

int qw6_fail(const char* fmt, ...);

}  // namespace qw6
