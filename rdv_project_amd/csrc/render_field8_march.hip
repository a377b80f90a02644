// The 8-tile instantiations of raymarch_generic_kernel (RaymarchingTransmittance
// with a runtime-shaped extinction): render.hip compiled with RDV_FIELD_PART 1,
// which emits only their launcher. They take most of render.hip's compile time;
// as a unit of their own they build in parallel with it.
#define RDV_FIELD_PART 1
#include "render.hip"
