// stubs.cpp -- the reference's out-of-scope launchers, exported so that the
// reference's loaders bind every symbol they expect (kernel_craft_torch_ops.py
// :101-168 binds launch_flash_attention, launch_paged_attention and
// launch_verify_draft_tokens for every op; pybind_transformer.cpp:36-122
// links the rest).  Each stub launches nothing, prints one line to stderr and
// records KC_ERR_NOT_IMPLEMENTED; the NCCL queries return the values of the
// reference's own no-NCCL stubs (tensor_parallel_nccl.cu:196-197).
#include <cstdio>

#include "kc_common.hpp"

namespace {
void stub(const char* name) {
    std::fprintf(stderr, "[kernel-craft-hip stub] %s not implemented\n", name);
    kc::set_error(KC_ERR_NOT_IMPLEMENTED, "%s not implemented", name);
}
}  // namespace

extern "C" {

void launch_flash_attention(const float*, const float*, const float*, float*, int, int, int, int,
                            int, bool, kc_stream_t) {
    stub("launch_flash_attention");
}

void launch_paged_attention(const float*, const int*, const float*, const float*, float*,
                            const int*, int, int, int, int, int, int, kc_stream_t) {
    stub("launch_paged_attention");
}

void launch_verify_draft_tokens(const float*, const float*, const int*, const float*,
                                const float*, int*, int*, int, int, kc_stream_t) {
    stub("launch_verify_draft_tokens");
}

void launch_compute_prefix_length(const int*, int*, int, kc_stream_t) {
    stub("launch_compute_prefix_length");
}

void launch_ring_allreduce(float**, int, int, kc_stream_t) { stub("launch_ring_allreduce"); }

void launch_allgather(float**, float*, int, int, kc_stream_t) { stub("launch_allgather"); }

void launch_col_parallel_linear(const float*, const float*, float*, int, int, int, kc_stream_t) {
    stub("launch_col_parallel_linear");
}

void launch_row_parallel_linear(const float*, const float*, float*, int, int, int, kc_stream_t) {
    stub("launch_row_parallel_linear");
}

void launch_selective_scan(const float*, const float*, const float*, const float*, const float*,
                           float*, int, int, int, int, kc_stream_t) {
    stub("launch_selective_scan");
}

void launch_depthwise_conv1d(const float*, const float*, const float*, float*, int, int, int, int,
                             kc_stream_t) {
    stub("launch_depthwise_conv1d");
}

void nccl_comm_init_all(void**, int, const int*) { stub("nccl_comm_init_all"); }
void nccl_comm_destroy(void*) {}
void nccl_group_start(void) {}
void nccl_group_end(void) {}

void launch_ring_allreduce_nccl(void*, float*, int, kc_stream_t) {
    stub("launch_ring_allreduce_nccl");
}

void launch_allgather_nccl(void*, const float*, float*, int, kc_stream_t) {
    stub("launch_allgather_nccl");
}

int nccl_comm_count(void*) { return 0; }
int nccl_comm_user_rank(void*) { return -1; }

}  // extern "C"
