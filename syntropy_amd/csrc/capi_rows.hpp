// The provider's forms of the C API's entries: the same calls with `active`, the device address
// of a step descriptor's rows_active (crates/kernels/include/syntropy/step_desc.h:53-57), or
// null for the whole bucket.  The kernels read it on the device, so a captured launch follows
// the value the host writes before each replay; rows past it are neither computed nor written.
// syn_moe_grouped_rows' `report`, when given, is three words of host-visible memory: the first
// refused launch (an id that names no expert) writes 1 + the slot, the id and top_k, if word 0
// is clear.  Its `layout` is the experts' (0 GGUF order, 3 TILE64 for Q4_K).
#pragma once

#include <stdint.h>

int syn_gemv_layout_rows(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                         uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
                         void* stream, const uint32_t* active);
int syn_gate_up_act_rows(uint32_t layout, int32_t wtype, const void* w, uint64_t w_bytes, uint32_t n_out,
                         uint32_t k_in, const float* x, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
                         void* stream, const uint32_t* active);
int syn_logits_rows(uint32_t layout, int32_t wtype, const void* head, uint64_t head_bytes, uint32_t vocab,
                    uint32_t hidden, const float* g, float eps, const float* x, uint32_t rows, float* y, void* ws,
                    uint64_t ws_bytes, void* stream, const uint32_t* active);
int syn_moe_route_rows(const float* router, const float* x, uint32_t rows, uint32_t hidden, uint32_t n_experts,
                       uint32_t top_k, int32_t renormalize, int32_t* ids, float* w, float* probs, void* stream,
                       const uint32_t* active);
int syn_moe_grouped_rows(int32_t wtype, const void* gate, const void* up, const void* down,
                         uint64_t expert_bytes_each, uint32_t n_experts, uint32_t top_k, uint32_t hidden,
                         uint32_t inter, const float* x, const int32_t* ids, const int32_t* site, uint32_t rows,
                         float* out, void* ws,
                         uint64_t ws_bytes, uint32_t* status, void* stream, const uint32_t* active,
                         uint32_t* report = nullptr, uint32_t layout = 0);
int syn_moe_combine_rows(const float* out, const int32_t* ids, const float* w, uint32_t rows, uint32_t top_k,
                         uint32_t hidden, float* y, void* stream, const uint32_t* active);
int syn_moe_combine_ranked_rows(const float* out, const float* w, uint32_t n_shared, const float* const* shared,
                                uint32_t rows, uint32_t top_k, uint32_t hidden, float* y, void* stream,
                                const uint32_t* active);
