// kk_host.h -- host-only rules of the library: the ragged layout tables, the duration rule and the
// checks of an ids-level item.  No HIP in these files (kk_host.cpp), so the same source also builds
// with a plain C++ compiler under AddressSanitizer / UndefinedBehaviorSanitizer for the CPU tests.
#pragma once
#include <cstdint>
#include <string>

#include "kokoro_hip.h"

namespace kk {

constexpr int kGapN = 2;  // GAP_N (src/gpu_batch.rs:27): gap frames after each item
constexpr int kGapT = 2;  // GAP_T (src/gpu_batch.rs:29): gap token rows after each item

// The refusal of one ids-level item (src/gpu_batch.rs:182-187: null inputs, input_ids length
// outside [2, 512], an id outside the vocabulary, speed not positive and finite, an unknown noise
// kind), or "" for an item the forward accepts.  The fixed noise's length is checked against the
// predicted frames later.
std::string ids_item_error(const kk_item& it, int b);

}  // namespace kk
