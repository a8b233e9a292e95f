// Drop-in for src/layers/seedvr2_dit_block.h of the reference: the same
// class name, debug struct and creator, with the block running in
// libseedvr2_hip (sv2::DiTBlockLayer over ncnn's types).  Built inside an
// ncnn build tree (include path of ncnn's layer.h and this repository's
// include/), linked against libseedvr2_hip.so.
#pragma once

#include <layer.h>

#include "seedvr2_dit_block_layer.h"

struct Sv2NcnnApi
{
    using Layer = ncnn::Layer;
    using ParamDict = ncnn::ParamDict;
    using ModelBin = ncnn::ModelBin;
    using Mat = ncnn::Mat;
    using Option = ncnn::Option;
};

// seedvr2_dit_block.h:20-36
typedef sv2::BlockDebugTensors<ncnn::Mat> SeedVR2DiTBlockDebugTensors;

// seedvr2_dit_block.h:38-170
class SeedVR2DiTBlock : public sv2::DiTBlockLayer<Sv2NcnnApi>
{
};

// seedvr2_dit_block.h:172
ncnn::Layer* SeedVR2DiTBlock_layer_creator(void* userdata);
