// Everything a user of the hot path includes.
#pragma once

#include "mensurflow/device.hpp"
#include "mensurflow/dtype.hpp"
#include "mensurflow/execution.hpp"
#include "mensurflow/ops/attention.hpp"
#include "mensurflow/ops/blas.hpp"
#include "mensurflow/ops/elementwise.hpp"
#include "mensurflow/ops/random.hpp"
#include "mensurflow/ops/reduction.hpp"
#include "mensurflow/ops/softmax.hpp"
#include "mensurflow/shape.hpp"
#include "mensurflow/tensor.hpp"
#include "mensurflow/trace.hpp"
