// Where an op runs, chosen per call (the reference's include/mensurflow/execution.hpp):
//   CPU   on the CPU;
//   GPU   on the GPU the inputs live on, otherwise the first available GPU (CUDA, Metal,
//         ROCm); runtime_error if there is none;
//   Auto  the CPU (no tuner in this build).
// When the data lives elsewhere, inputs are copied to the execution device and results back.
#pragma once

namespace mensurflow {

enum class Execution { Auto, CPU, GPU };

const char* execution_name(Execution execution);

} // namespace mensurflow
