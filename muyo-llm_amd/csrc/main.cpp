// muyo_llm: the reference CLI (src/main.cpp) on the gfx950 kernels.
//
//   muyo_llm [--smoke | --add | --matvec | --rmsnorm | --rope | --swiglu | --getrows | --argmax |
//             --softmax | --attention | --kvcache]
//   muyo_llm --tokenize <gguf> <text>
//   muyo_llm --forward <gguf> [-p <text> | --tokens id,id] [-n N] [--temp T] [--top-k K] [--top-p P]
//            [--repeat-penalty R] [--repeat-last-n N] [--seed S] [--chat] [-i] [--system <text>]
//            [--ctx N]
//
// The self-test modes (src/main.cpp:188-310) run each kernel against a CPU reference; --smoke runs
// them all. --tokenize and --forward (src/main.cpp:209-226, 309-423) are in forward.cpp.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

#include "muyo_hip.h"

extern "C" int muyo_self_test(const char* mode);

int RunForward(int argc, char** argv);
int RunTokenize(const char* path, const char* text);

int main(int argc, char** argv)
{
    const char* mode = argc > 1 ? argv[1] : "--smoke";
    // --tokenize reads the GGUF tokenizer and needs no device.
    if (std::strcmp(mode, "--tokenize") == 0)
    {
        if (argc < 4)
        {
            std::fprintf(stderr, "usage: %s --tokenize <gguf> <text>\n", argv[0]);
            return 2;
        }
        return RunTokenize(argv[2], argv[3]);
    }
    // --forward checks its flags before it looks for a device.
    if (std::strcmp(mode, "--forward") == 0)
    {
        return RunForward(argc, argv);
    }
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
