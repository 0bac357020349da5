// raggedroute/raggedroute.h - umbrella header for the C++ v0.2 surface.
#pragma once

#include "raggedroute/baseline_ops.h"
#include "raggedroute/chain.h"
#include "raggedroute/dispatch.h"
#include "raggedroute/operators.h"
#include "raggedroute/runtime.h"
#include "raggedroute/status.h"
#include "raggedroute/types.h"
