// The launcher of the 8-tile instantiations of volume_profile_dda_kernel
// (VolumeProfileDDA): volume_profile.hip compiled with RDV_FIELD_PART 3, which
// emits only that. As a unit of its own it builds in parallel with the others.
#define RDV_FIELD_PART 3
#include "volume_profile.hip"
