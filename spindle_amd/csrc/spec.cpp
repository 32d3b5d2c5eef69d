// C entry points over the speculative loop's draft-length model (spec.h), the same object the
// engine's generate loop drives, so a host can keep its own loop or test the model directly.
#include <new>

#include "../../include/spx.h"
#include "spec.h"

struct spx_spec_model {
  spx::SpecModel m;
};

extern "C" {

spx_spec_model *spx_spec_create(int fixed) {
  spx_spec_model *s = new (std::nothrow) spx_spec_model();
  if (s) s->m.fixed = fixed != 0;
  return s;
}

spx_spec_model *spx_spec_clone(const spx_spec_model *s) { return s ? new (std::nothrow) spx_spec_model(*s) : nullptr; }

void spx_spec_destroy(spx_spec_model *s) { delete s; }

int spx_spec_class(int ngram) { return spx::SpecModel::cls(ngram); }

static bool bad_class(int c) { return c < 0 || c > 3; }

double spx_spec_accept_rate(const spx_spec_model *s, int c) { return !s || bad_class(c) ? -1.0 : s->m.rate(c); }

int spx_spec_best_len(spx_spec_model *s, int c, int avail) {
  if (!s || bad_class(c) || avail < 0) return -1;
  return s->m.best_len(c, avail);
}

void spx_spec_reset_rates(spx_spec_model *s) {
  if (s) s->m.reset_rates();
}

int spx_spec_record_draft(spx_spec_model *s, int c, int drafted, int accepted) {
  if (!s || bad_class(c) || drafted < 0 || accepted < 0 || accepted > drafted) return -1;
  s->m.record_draft(c, drafted, accepted);
  return 0;
}

void spx_spec_record_step(spx_spec_model *s, uint64_t us) {
  if (s) s->m.record_step(us);
}

void spx_spec_record_verify(spx_spec_model *s, int b, uint64_t us) {
  if (s) s->m.record_verify(b, us);
}

}  // extern "C"
