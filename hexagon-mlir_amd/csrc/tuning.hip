// Launch-shape tuning knobs: process-wide values read once from the
// environment (HXMI_<NAME>) when the library is loaded, plus per-thread
// overrides set through hxmi_set_tuning.  Every knob only changes how a
// result is computed (tile shape, K split, kernel choice), never the
// result's definition; the dispatchers call knob() on each launch, which is
// a thread-local read.
#include <limits.h>
#include <stdlib.h>
#include <string.h>

#include "hxmi_internal.h"

namespace hxmi {
namespace {

struct KnobInfo {
  const char* name;  // hxmi_set_tuning name; the variable is HXMI_ + upper case
  const char* env;
};

constexpr KnobInfo kKnobs[KNOB_COUNT] = {
    {"gemm_tile", "HXMI_GEMM_TILE"}, {"group_m", "HXMI_GROUP_M"},     {"splitk", "HXMI_SPLITK"},
    {"w8_tile", "HXMI_W8_TILE"},     {"gemv_path", "HXMI_GEMV_PATH"}, {"gemv_tpb", "HXMI_GEMV_TPB"},
    {"gemv_ks", "HXMI_GEMV_KS"},     {"gemv_kg", "HXMI_GEMV_KG"},     {"gemv_unr", "HXMI_GEMV_UNR"},
    {"gemv_pair_wg", "HXMI_GEMV_PAIR_WG"}, {"attn_cfg", "HXMI_ATTN_CFG"},
};

int64_t g_env[KNOB_COUNT];
thread_local int64_t t_over[KNOB_COUNT] = {KNOB_UNSET, KNOB_UNSET, KNOB_UNSET, KNOB_UNSET,
                                           KNOB_UNSET, KNOB_UNSET, KNOB_UNSET, KNOB_UNSET,
                                           KNOB_UNSET, KNOB_UNSET, KNOB_UNSET};
static_assert(KNOB_COUNT == 11, "t_over initialiser");

// HXMI_GEMV_PATH names a kernel by its first letter: valu, pair, k-split
// pair; anything else is the 16-row MFMA kernel
int64_t parse(int k, const char* v) {
  if (k == KNOB_GEMV_PATH) return v[0] == 'v' ? GEMV_PATH_VALU : v[0] == 'p' ? GEMV_PATH_PAIR
                                  : v[0] == 'k' ? GEMV_PATH_PAIR_KS : GEMV_PATH_MFMA;
  return atoll(v);
}

__attribute__((constructor)) void read_environment() {
  for (int k = 0; k < KNOB_COUNT; ++k) {
    const char* v = getenv(kKnobs[k].env);
    g_env[k] = v && v[0] ? parse(k, v) : KNOB_UNSET;
  }
}

}  // namespace

int64_t knob(Knob k) { return t_over[k] != KNOB_UNSET ? t_over[k] : g_env[k]; }

int knob_index(const char* name) {
  if (!name) return -1;
  for (int k = 0; k < KNOB_COUNT; ++k)
    if (strcmp(name, kKnobs[k].name) == 0) return k;
  return -1;
}

int64_t set_knob_override(int k, int64_t value) {
  const int64_t prev = t_over[k];
  t_over[k] = value < 0 ? KNOB_UNSET : value;
  return prev == KNOB_UNSET ? -1 : prev;
}

}  // namespace hxmi
