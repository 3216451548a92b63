// fa_bwd.hip - placeholder table until the backward kernels land.
#include "fa_device.h"
#include "fa_launch.h"

extern "C" FA_HIDDEN fa::BwdFn FA_BWD_TABLE(int bm, int bn) {
  (void)bm; (void)bn;
  return nullptr;
}
