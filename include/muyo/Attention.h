#pragma once

namespace muyo_llm
{
/// Run single-head attention as score GEMV, softmax and value GEMV over 16 keys and verify it
/// against a CPU reference (src/Attention.h).
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunAttention();
}  // namespace muyo_llm
