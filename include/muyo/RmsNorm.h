#pragma once

namespace muyo_llm
{
/// Run rms_norm (`y = x * rsqrt(mean(x^2) + eps) * weight`) over 8 rows of 512 and verify it
/// against a CPU reference within 1e-4 relative (src/RmsNorm.h).
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunRmsNorm();
}  // namespace muyo_llm
