// wzy_stage_int.h -- library-internal hooks of the stage for its loaders (not part of the C ABI).
#pragma once
#include "../../include/wzy_stage.h"

namespace wzy {

const wzy_stage_cfg* stage_cfg(const wzy_stage* st);
// loaded = false while a loader writes the weights; loaded = true also empties the recurrent state
// (as wzy_stage_reset_state) and waits for the stage stream
int stage_set_loaded(wzy_stage* st, bool loaded);
// free the drafter (a loader that failed half way)
void stage_mtp_drop(wzy_stage* st);

}  // namespace wzy
