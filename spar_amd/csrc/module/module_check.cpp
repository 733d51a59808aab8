// A consumer of the spar.hip_ops module: imports it, calls launchers through
// it and reports what came back.  Needs no GPU: a zero-element launch returns
// success before touching a device, and a bad element type is rejected on
// the host with SPAR_HIP_STATUS 1, which the module turns into
// std::invalid_argument.
#include <cstdio>
#include <stdexcept>

import spar.hip_ops;

int main() {
  namespace ops = spar::detail::hip_ops;
  ops::binary(nullptr, nullptr, nullptr, 0, ops::ElementType::Float32,
              ops::BinaryOperation::Add, 0);
  bool rejected = false;
  try {
    ops::binary(nullptr, nullptr, nullptr, 4, static_cast<ops::ElementType>(7),
                ops::BinaryOperation::Add, 0);
  } catch (const std::invalid_argument&) {
    rejected = true;
  }
  std::printf("spar.hip_ops: empty launch ok, invalid dtype %s, %d HIP device(s)\n",
              rejected ? "rejected" : "NOT rejected", ops::device_count());
  return rejected ? 0 : 1;
}
