#pragma once

namespace muyo_llm
{
/// Run the row argmax over planted logits and verify the index (src/Argmax.h). Ties resolve
/// to the lowest index.
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunArgmax();
}  // namespace muyo_llm
