// Internal interface of the fused MoE-layer kernels (cw_moe_fused.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cw {

struct MoeArgs {
    const uint8_t *wg, *wu, *wd;   // gate, up, down banks
    int64_t sg, su, sd;            // slot strides (bytes)
    int64_t rbg, rbd;              // bytes per row of gate/up and of down
    int E, K, H, I, P;             // experts, top-k, hidden, inter, down's row width (>= I)
    int n_slots;
    int norm, act;
    float alpha, limit;
    const float *bg, *bu, *bd;     // biases (E x I, E x I, E x H) or NULL
    const uint32_t *table;         // expert -> slot, or NULL (slot = expert)
    uint32_t *missing;             // picks without a slot, or NULL
    const float *x;                // T x H
    const float *logits;           // T x E
    uint32_t *ids;                 // T x K experts (written by the gate/up kernel)
    float *w;                      // T x K weights
    uint32_t *slots;               // T x K slots
    float *h;                      // T*K x P hidden rows
    float *out;                    // T x H
    void *state;                   // the one-launch decode's sync state (DECODE_STATE_BYTES, zero-
                                   // filled before the first call; each call leaves it valid)
    uint32_t polls;                // its bounded waits give up after this many polls
    int per_cu;                    // blocks per CU of the one-launch decode (set by its launch)
};

// workspace bytes of the decode's sync state, at the start of every MoE-layer workspace: the
// barrier (8 KB), a word that tells a valid state from foreign bytes, and the status word
// (CW_MOE_STATUS_OFFSET)
constexpr size_t DECODE_STATE_BYTES = 8192 + 256;

int moe_gateup(int dtype, const MoeArgs &a, int T, hipStream_t s);
// the whole layer for one token in one launch (CW_ENOTSUP for shapes it does not cover)
int moe_decode(int dtype_gate_up, int dtype_down, const MoeArgs &a, hipStream_t s);
uint32_t decode_barrier_errors();
int moe_down(int dtype, const MoeArgs &a, int T, hipStream_t s);

}  // namespace cw
