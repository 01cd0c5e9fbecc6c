#pragma once

namespace muyo_llm
{
/// Run get_rows (an embedding lookup) and verify the gathered row bit-exactly (src/GetRows.h).
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunGetRows();
}  // namespace muyo_llm
