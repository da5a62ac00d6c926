// helix_kernels.hip -- the one translation unit compiled to the gfx950 code
// object embedded in libhelix.so. Kernel names are resolved by the runtime
// (helix_amd/csrc/runtime/caps.cpp traits tables).
#include "pass_a_x6.hip"
#include "pass_a_hb.hip"
#include "pass_b.hip"
#include "pass_c_f32.hip"
#include "pass_c_x6.hip"
#include "pass_c_walk16.hip"
#include "pass_c_walk_x6.hip"
#include "pass_single.hip"
