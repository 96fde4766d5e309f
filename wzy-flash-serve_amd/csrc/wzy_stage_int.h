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
// the per-layer embedding table of a cfg.ple stage: not ready (a load begins), or ready with its scale;
// a stage runs no forward while its table is not ready
int stage_set_ple_table(wzy_stage* st, bool ready, float scale);

}  // namespace wzy
