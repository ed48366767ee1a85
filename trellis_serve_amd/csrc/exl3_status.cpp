// Status and last-error plumbing of the C-ABI (one copy per process).
#include <string>

#include "exl3_api.hpp"

namespace exl3 {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

}  // namespace exl3

extern "C" const char* exl3_last_error(void) { return exl3::g_last_error.c_str(); }

extern "C" int exl3_abi_version(void) { return EXL3_ABI_VERSION; }

extern "C" int exl3_init_device(int device) {
  int count = 0;
  EXL3_CHECK_HIP(hipGetDeviceCount(&count));
  EXL3_CHECK_ARG(device >= 0 && device < count, "exl3_init_device: device %d out of range (%d devices)", device, count);
  hipDeviceProp_t prop;
  EXL3_CHECK_HIP(hipGetDeviceProperties(&prop, device));
  if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
    return exl3::set_error(EXL3_ERR_UNSUPPORTED, "exl3_init_device: device %d is %s, this library is built for gfx950",
                           device, prop.gcnArchName);
  return exl3::xcd_probe(device);
}
