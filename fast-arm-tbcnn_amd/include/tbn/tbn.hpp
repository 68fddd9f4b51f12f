// Umbrella header of the tbn host runtime on the MI355X
// (the reference's tbn-runtime/include/tbn/tbn.hpp).
#pragma once

#include "device.hpp"
#include "errors.hpp"
#include "model.hpp"
#include "onnx_parser.hpp"
#include "operators.hpp"
#include "session.hpp"
#include "tensor.hpp"
#include "types.hpp"
