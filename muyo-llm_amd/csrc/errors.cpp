// Per-thread error message storage behind muyo_last_error().
#include <cstdarg>
#include <cstdio>
#include <string>

#include "common.hpp"

namespace muyo
{
namespace
{
thread_local std::string g_lastError;

void Format(const char* format, va_list args)
{
    char buffer[512];
    std::vsnprintf(buffer, sizeof buffer, format, args);
    g_lastError = buffer;
}
}  // namespace

void SetLastError(const char* format, ...)
{
    va_list args;
    va_start(args, format);
    Format(format, args);
    va_end(args);
}

void ClearLastError() { g_lastError.clear(); }

int Fail(int code, const char* format, ...)
{
    va_list args;
    va_start(args, format);
    Format(format, args);
    va_end(args);
    return code;
}

int HipStatus(hipError_t status, const char* what)
{
    SetLastError("%s failed: %s (%d)", what, hipGetErrorString(status), static_cast<int>(status));
    return static_cast<int>(status);
}
}  // namespace muyo

extern "C" const char* muyo_last_error(void) { return muyo::g_lastError.c_str(); }

extern "C" const char* muyo_version(void) { return "muyo_hip 0.1 (gfx950)"; }
