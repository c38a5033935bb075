// Internal declarations shared by the engine's translation units.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "bsscl_hip.h"

namespace bsscl {

// Records `msg` as the calling thread's last error and returns `code`.
int set_error(int code, const std::string &msg);

// Sampler hand-off used by bsscl_boost_round (sampler.cpp).
int sampler_take(bsscl_sampler *s, const int32_t **rows, const int32_t **feats,
                 void **token);
void sampler_give_back(bsscl_sampler *s, void *token);
int64_t sampler_n_sub(bsscl_sampler *s);
int32_t sampler_f_sub(bsscl_sampler *s);

}  // namespace bsscl
