#pragma once

namespace muyo_llm
{
/// Run `d = silu(gate) * up` (split mode) and verify it against a CPU reference (src/Swiglu.h).
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunSwiglu();
}  // namespace muyo_llm
