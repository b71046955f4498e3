// The decoder's public types live in include/trixium.h.
#pragma once
#include "../../include/trixium.h"
