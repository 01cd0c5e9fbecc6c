#pragma once

namespace muyo_llm
{
/// Run the element-wise add `d = a + b` and verify it bit-exactly (src/ElementwiseAdd.h).
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunElementwiseAdd();
}  // namespace muyo_llm
