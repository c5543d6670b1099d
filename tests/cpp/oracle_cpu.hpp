// Test-only: CPU kernels for the host layer's dispatcher, served by the C oracle
// (oracle/liboracle.so, a restatement of the reference's CPU kernels). In a real mensurflow build
// the reference's own CPU backend provides these; the product library registers none.
#pragma once

namespace test {

// Registers {Matmul, GemmBatched, Gemv, Matvec, BiasAdd, Gelu, Where, Softmax, Argmax, Add, Mul,
// Scal, Uniform, Normal} x {CPU, F32}. Call once, before the first op.
void register_oracle_cpu_kernels();

} // namespace test
