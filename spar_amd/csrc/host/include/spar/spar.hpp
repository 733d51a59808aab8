// Umbrella header of the host library (the counterpart of `import spar;`,
// src/spar.cppm:1-15, for the tensor/ops path this backend covers).
#pragma once

#include "spar/core.hpp"
#include "spar/loss.hpp"
#include "spar/ops.hpp"
#include "spar/optim.hpp"
#include "spar/random.hpp"
#include "spar/tensor.hpp"
