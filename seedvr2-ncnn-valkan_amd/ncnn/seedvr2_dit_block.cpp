// Drop-in for src/layers/seedvr2_dit_block.cpp of the reference (the layer's
// creator, seedvr2_dit_block.cpp:1681); everything else is in
// seedvr2_dit_block_layer.h and libseedvr2_hip.so.
#include "seedvr2_dit_block.h"

DEFINE_LAYER_CREATOR(SeedVR2DiTBlock)
