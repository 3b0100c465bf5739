// Internal declarations shared by the GEMM translation units.
#pragma once

#include "../../include/voyager_hip.h"
