// Internal helpers shared by the translation units of libsf_rdt.so.
#pragma once

#include <string>

#include "sf_rdt.h"

// Records the message sf_rdt_last_error returns for this model.
void sf_rdt_set_error(sf_rdt* m, const std::string& msg);

// New parameter values were written: the condition sf_rdt_infer cached was
// encoded with the old ones.
void sf_rdt_weights_changed(sf_rdt* m);
