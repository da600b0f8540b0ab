// Library-level entry points of libmentat_hip.so (version and device queries).
#include "mentat_common.h"

extern "C" int mentat_abi_version(void) { return 6; }

extern "C" int mentat_device_count(void) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return -(int)e;
  return n;
}
