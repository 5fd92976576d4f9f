// CPU stand-in (see hip_runtime.h beside this file).
#pragma once
#include "hip_runtime.h"
