// The 8-tile instantiations of ratiotracking_generic_kernel (ratio tracking):
// render.hip compiled with RDV_FIELD_PART 2, which emits only their launcher.
// They take most of render.hip's compile time; as a unit of their own they build
// in parallel with it.
#define RDV_FIELD_PART 2
#include "render.hip"
