// Test-side declaration of moss::SampleParams for building the GPU LlmModel shim
// where the reference's csrc/include/moss/sampler.h is not on the include path.
// Same fields, order and defaults as that header's SampleParams (sampler.h:8-22);
// an integration build uses the reference's own header instead of this one.
#pragma once

namespace moss {

struct SampleParams {
    bool greedy = true;
    float temperature = 1.0f;
    int top_k = 0;
    float top_p = 1.0f;
    float repetition_penalty = 1.0f;
    bool end_greedy = true;
    int min_frames = 0;
    int greedy_frames = 0;
};

}  // namespace moss
