// Grid i-quants (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M): not built yet.
#include "launch.h"

namespace spa {
int launch_iqgrid(const QuantArgs& a) { return fail(-2, "grid i-quant type %d not built yet", a.type); }
}  // namespace spa
