// Umbrella header of the VeloMind API subset built here (the quantized
// linear layer path on DeviceType::HIP).
#pragma once

#include "velomind/types.h"
#include "velomind/device.h"
#include "velomind/dtype.h"
#include "velomind/ptr.h"
#include "velomind/tensor_storage.h"
#include "velomind/tensor.h"
#include "velomind/ops.h"
#include "velomind/node.h"
#include "velomind/executable.h"
#include "velomind/graph.h"
#include "velomind/quant.h"
