#pragma once

namespace muyo_llm
{
/// Run NeoX rope (pairs (j, j + nDims/2), theta = pos * thetaScale^j) and verify it against a
/// CPU reference (src/Rope.h).
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunRope();
}  // namespace muyo_llm
