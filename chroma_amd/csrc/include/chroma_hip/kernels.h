// Umbrella header included by every generated model.hip of the hip backend.
#pragma once

#include "device.h"
#include "linear.h"
#include "attention.h"
