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
/// Default system text (Qwen2.5's own template uses it whenever a chat names no system turn).
inline constexpr char QWEN2_DEFAULT_SYSTEM[] = "You are Qwen, created by Alibaba Cloud. You are a helpful assistant.";

/// Frames `system` as ChatML's system block, ending on a newline.
inline std::string Qwen2SystemStart(const std::string& system)
{
    return "<|im_start|>system\n" + system + "<|im_end|>\n";
}

/// Frames `user` as a user block, then opens the assistant block the model continues.
inline std::string Qwen2UserTurn(const std::string& user)
{
    return "<|im_start|>user\n" + user + "<|im_end|>\n<|im_start|>assistant\n";
}

/// A whole first exchange: the system block followed by the user block and the open assistant block.
inline std::string Qwen2ChatStart(const std::string& system, const std::string& user)
{
    return Qwen2SystemStart(system) + Qwen2UserTurn(user);
}
}  // namespace chat_template
}  // namespace hip
}  // namespace muyo_llm
