#pragma once
// Declarations of TensorPlay's host generator as the reference uses it
// (tensorplay_mlu/csrc/NNKernels.cpp:181-183), for the adapter's syntax
// check; nothing here is linked.
#include <cstdint>

namespace tensorplay {
class Generator {
public:
    uint64_t random64();
};
Generator& default_generator();
}  // namespace tensorplay
