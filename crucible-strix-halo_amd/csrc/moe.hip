// MoE layer path (route, group, expert GEMMs, combine).
#include "internal.hpp"

extern "C" {
int cx_moe_route(const float*, int32_t, int32_t, int32_t, int32_t, const float*, int32_t*, float*, cx_stream_t) {
  return CX_E_UNSUPPORTED;
}
size_t cx_moe_group_workspace_size(int32_t, int32_t, int32_t) { return 0; }
int cx_moe_group(const int32_t*, int32_t, int32_t, int32_t, int32_t*, int32_t*, int32_t*, int32_t*, void*, size_t,
                 cx_stream_t) {
  return CX_E_UNSUPPORTED;
}
int cx_moe_plan_create(const cx_moe_layer*, cx_moe_plan**) { return CX_E_UNSUPPORTED; }
void cx_moe_plan_destroy(cx_moe_plan*) {}
size_t cx_moe_layer_workspace_size(const cx_moe_plan*, int32_t, int32_t) { return 0; }
int cx_moe_layer_forward(const cx_moe_plan*, const uint16_t*, const float*, int32_t, const float*, int32_t,
                         const int32_t*, int32_t, float*, int32_t*, float*, int32_t, void*, size_t, cx_stream_t) {
  return CX_E_UNSUPPORTED;
}
}
