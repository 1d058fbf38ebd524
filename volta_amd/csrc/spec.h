// Internal helpers around volta_mlp_spec (shared by the HIP library and the
// CPU oracle).
#pragma once

#include <string>
#include <vector>

#include "../../include/volta_train.h"

namespace volta {

void set_last_error(const std::string& msg);
const char* last_error();
bool validate_spec(const volta_mlp_spec& s, std::string* why);
const char* activation_name(int a);
const char* optimizer_name(int o);

// Process-wide default spec for volta_train_init(batch): the one given to
// volta_train_configure, else VOLTA_MLP_SPEC parsed from the environment.
bool resolve_default_spec(volta_mlp_spec* out);

}  // namespace volta
