// Placeholder launchers for the i-quant families until their kernels land.
#include "launch.h"

namespace spa {
int launch_iq4(const QuantArgs& a) { return fail(-2, "IQ4 type %d not built yet", a.type); }
int launch_iqgrid(const QuantArgs& a) { return fail(-2, "grid i-quant type %d not built yet", a.type); }
}  // namespace spa
