// muyo_llm: the reference CLI's self-test modes (src/main.cpp:188-310) on the gfx950 kernels.
//
//   muyo_llm [--smoke | --add | --matvec | --rmsnorm | --rope | --swiglu | --getrows | --argmax |
//             --softmax | --attention | --kvcache]
//
// --smoke runs every self-test. The GGUF, tokenizer and --forward generation modes of the
// reference are not part of this library (the decode step is reached through muyo_decoder_*).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

#include "muyo_hip.h"

extern "C" int muyo_self_test(const char* mode);

int main(int argc, char** argv)
{
    const char* mode = argc > 1 ? argv[1] : "--smoke";
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0)
    {
        std::fprintf(stderr, "[fail] no HIP device\n");
        return 1;
    }
    std::printf("[muyo_llm] %s, mode %s\n", muyo_version(), mode);
    const int status = muyo_self_test(mode);
    if (status == MUYO_E_RANGE)
    {
        std::fprintf(stderr,
                     "unknown mode %s (expected --smoke, --add, --matvec, --rmsnorm, --rope, --swiglu, --getrows, "
                     "--argmax, --softmax, --attention or --kvcache)\n",
                     mode);
        return 2;
    }
    return status == 0 ? 0 : 1;
}
