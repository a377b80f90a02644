// The 8-tile instantiations of render_ea_generic_kernel (emission-absorption
// with a runtime-shaped field): render.hip compiled with RDV_FIELD_PART 3, which
// emits only their launcher. They take most of render.hip's compile time; as a
// unit of their own they build in parallel with it.
#define RDV_FIELD_PART 3
#include "render.hip"
