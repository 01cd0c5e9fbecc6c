#pragma once

namespace muyo_llm
{
/// Append roped keys and values to a KV cache over two tokens with the per-op nodes (rope into
/// the key cache, value-column copy, score GEMV, softmax, value GEMV) and verify the attention
/// output against a CPU reference after each append (src/KvCache.h).
///
/// Needs a HIP device; runs on the current one.
/// @return 0 when the GPU result matches the CPU reference, 1 otherwise.
int RunKvCache();
}  // namespace muyo_llm
