// Host-only helpers (no HIP headers) for the plain C++ sources of the library.
#pragma once

#include "vlc_capi.h"

#define VLC_HOST_API extern "C" __attribute__((visibility("default")))
