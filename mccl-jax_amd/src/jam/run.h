// jam runtime: executes a launch plan on one device stream.
//
// Replaces jam::Run (src/jam/jam_run.h:15-40, jam_run.mm:361-419).  Same
// contract — validate inputs, acquire output buffers, run — but nothing
// blocks: the launches are queued on the device context's stream and the
// caller records an event after them.
#pragma once

#include <string>
#include <vector>

#include "execution/device.h"
#include "jam/program.h"

namespace mi::jam {

struct RunInput {
  const void* data = nullptr;  // device pointer
  size_t nbytes = 0;
};

struct RunOutput {
  void* data = nullptr;        // device pointer owned by the caller afterwards (DeviceContext::Free)
  size_t nbytes = 0;
  TensorType type;
};

// Queue every step of `prog` on dev.stream().  On error, returns a message
// prefixed "jam run:" and frees anything it allocated.  `preset` (optional,
// one entry per output) gives memory an output is written into instead of a
// fresh allocation: a donated input's buffer, for an output
// prog.input_alias names.  Run neither allocates nor frees preset memory.
std::string Run(Program& prog, exec::DeviceContext& dev, const std::vector<RunInput>& inputs,
                std::vector<RunOutput>& outputs, const std::vector<void*>* preset = nullptr);

}  // namespace mi::jam
