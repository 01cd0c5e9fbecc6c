#pragma once

namespace muyo_llm
{
/// Run the F16-weight GEMV (`mul_mat_vec_f16_f32_f32`) as `d[row] = sum_k A[row, k] * b[k]` on
/// the GPU and verify it against a CPU reference (src/MatVec.h). Exact: the inputs are small integers.
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunMatVec();
}  // namespace muyo_llm
