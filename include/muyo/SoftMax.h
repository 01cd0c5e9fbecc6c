#pragma once

namespace muyo_llm
{
/// Run the scaled row softmax and verify it against a CPU reference (src/SoftMax.h).
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunSoftMax();
}  // namespace muyo_llm
