// Launchers of the row kernels (rows.hip). All pointers are device memory; launchers return the kernel name.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace xtg::hip {

std::string launch_qk_rope_norm(float* q, float* k, int m, int heads, int kv_heads, int d, long long pos0,
                                const float* inv_freq, const float* qscale, hipStream_t stream);
std::string launch_slerp_norm(float* x, const float* o, const float* lr, int rows, int w, hipStream_t stream);
std::string launch_swiglu_norm(float* g, const float* u, const float* sg, const float* su, int rows, int w,
                               hipStream_t stream);
std::string launch_gate_norm(float* a, const float* gate, const float* gs, int rows, int w, hipStream_t stream);
std::string launch_add_norm(const float* a, const float* b, float* out, int rows, int w, hipStream_t stream);

}  // namespace xtg::hip
