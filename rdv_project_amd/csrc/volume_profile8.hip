// The 8-tile instantiations of volume_profile_kernel: volume_profile.hip
// compiled with RDV_FIELD_PART 1, which emits only their launcher. They take
// most of volume_profile.hip's compile time; as a unit of their own they build
// in parallel with it.
#define RDV_FIELD_PART 1
#include "volume_profile.hip"
