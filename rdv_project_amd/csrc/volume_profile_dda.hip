// The launcher of volume_profile_dda_kernel (VolumeProfileDDA) with 1, 2 and 4
// tiles, and its dispatch: volume_profile.hip compiled with RDV_FIELD_PART 2,
// which emits only that. As a unit of its own it builds in parallel with the
// others.
#define RDV_FIELD_PART 2
#include "volume_profile.hip"
