// esda_internal.h -- library-internal hooks shared by the HIP sources and the ES* C++
// layer (not part of the public ABI).
#pragma once
#include <string>

namespace esda_detail {
// Sets the calling thread's esda_last_error() message.
void set_error(const std::string &msg);
// ESDA_OK when the current device is a gfx950; otherwise sets the message and returns
// ESDA_ERR_DEVICE or ESDA_ERR_HIP.
int check_device();
}  // namespace esda_detail
