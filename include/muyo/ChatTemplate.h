#pragma once

// Qwen2.5's ChatML framing, as the reference writes it (src/ChatTemplate.h:9-29,
// src/ChatTemplate.cpp:9-31): literal pieces, fed to the tokenizer with special-token parsing on so
// that <|im_start|> and <|im_end|> become their own ids.

#include <string>

namespace muyo_llm
{
namespace hip
{
namespace chat_template
{
/// The system prompt Qwen2.5's template falls back to when none is given.
inline constexpr char QWEN2_DEFAULT_SYSTEM[] = "You are Qwen, created by Alibaba Cloud. You are a helpful assistant.";

/// "<|im_start|>system\n{system}<|im_end|>\n"
inline std::string Qwen2SystemStart(const std::string& system)
{
    return "<|im_start|>system\n" + system + "<|im_end|>\n";
}

/// "<|im_start|>user\n{user}<|im_end|>\n<|im_start|>assistant\n"
inline std::string Qwen2UserTurn(const std::string& user)
{
    return "<|im_start|>user\n" + user + "<|im_end|>\n<|im_start|>assistant\n";
}

/// The single-turn prompt: the system turn, then the user turn.
inline std::string Qwen2ChatStart(const std::string& system, const std::string& user)
{
    return Qwen2SystemStart(system) + Qwen2UserTurn(user);
}
}  // namespace chat_template
}  // namespace hip
}  // namespace muyo_llm
