// inferno.h -- umbrella header of the MI355X attention drop-in (cf. the reference's include/inferno/inferno.h).
#pragma once

#include "inferno/core/device.h"
#include "inferno/core/dtype.h"
#include "inferno/core/storage.h"
#include "inferno/core/tensor.h"
#include "inferno/core/tensorimpl.h"
#include "inferno/functional/attention.h"
#include "inferno/functional/softmax.h"
#include "inferno/gradengine/engine.h"
#include "inferno/gradfn/node.h"
