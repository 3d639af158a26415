// Launchers of the row kernels (rows.hip). All pointers are device memory; launchers return the kernel name.
// op (optional): also write the rows as a GEMV / GEMM activation operand (kernels.hpp layout: ceil(rows / 8) groups of
// Backend::op_bytes(w) bytes, each the operand of 8 rows, then their scales); w % 16 == 0 then.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace xtg::hip {

std::string launch_qk_rope_norm(float* q, float* k, int m, int heads, int kv_heads, int d, long long pos0,
                                const float* inv_freq, const float* qscale, hipStream_t stream);
// x = justnorm(slerp) in place; part (floats, optional): o is the sum of o and o + part (a K-split GEMV's two
// output sets, added in that order)
std::string launch_slerp_norm(float* x, const float* o, const float* lr, int rows, int w, void* op,
                              hipStream_t stream, size_t part = 0);
// out (optional, may be g) = justnorm(silu(g sg) (u su)); part as for slerp_norm, for g and u alike (out then may
// not be g or u)
std::string launch_swiglu_norm(const float* g, const float* u, const float* sg, const float* su, int rows, int w,
                               float* out, void* op, hipStream_t stream, size_t part = 0);
// out (optional, may be a) = justnorm(a sigmoid(gate gs))
std::string launch_gate_norm(const float* a, const float* gate, const float* gs, int rows, int w, float* out, void* op,
                             hipStream_t stream);
// out (may be a) = justnorm(a + b), b optional
std::string launch_add_norm(const float* a, const float* b, float* out, int rows, int w, void* op,
                            hipStream_t stream);
// out[r] = the first index of the largest of x[r][0 .. n) (xtg::argmax, sampler.cpp:8-13), int32 per row
std::string launch_argmax(const float* x, int rows, int n, int* out, hipStream_t stream);

}  // namespace xtg::hip
