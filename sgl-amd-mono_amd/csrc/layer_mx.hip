// The one-launch layer's MXFP4-expert instances (layer_kernel.h), compiled apart from the
// FP8 ones so the two sets build in parallel.
#include "layer_kernel.h"

namespace mono {

LayerKernel layer_kernel_mx(bool shuf, bool lng, bool dsa) {
  static const LayerKernel k[2][2][2] = {
      {{layer_kernel<false, 64, false, false, true>, layer_kernel<false, 64, false, true, true>},
       {layer_kernel<false, 64, true, false, true>, layer_kernel<false, 64, true, true, true>}},
      {{layer_kernel<true, 64, false, false, true>, layer_kernel<true, 64, false, true, true>},
       {layer_kernel<true, 64, true, false, true>, layer_kernel<true, 64, true, true, true>}}};
  return k[shuf][lng][dsa];
}

}  // namespace mono
