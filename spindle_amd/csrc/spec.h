// The adaptive draft-length model of the speculative loop (SpecModel, smollm_chat.rs:1670-1809):
// decayed accept counts per draft source and measured pass costs choose how many drafted tokens
// a verify pass takes. Host code; the engine's generate loop and the spx_spec_* entry points
// share this one definition.
#pragma once
#include <stdint.h>

#include <algorithm>

namespace spx {

struct SpecModel {
  double acc[4] = {1, 1, 1, 1}, fail_[4] = {1, 1, 1, 1};  // pseudo-counts per class (:1696-1697)
  double t1_us = 100000.0, extra_us = 30000.0;             // one-token step, each extra verify row
  bool have_t1 = false, have_extra = false, fixed = false;
  int since_try = 0;

  // Draft source class (:1710-1717): 0 = 2-gram lookup (n-gram 1 or 2), 1 = 3-gram,
  // 2 = 4+-gram, 3 = draft model (n-gram 0).
  static int cls(int ng) { return ng == 0 ? 3 : ng <= 2 ? 0 : ng == 3 ? 1 : 2; }
  double rate(int c) const { return acc[c] / (acc[c] + fail_[c]); }
  double cost(int b) const { return t1_us + extra_us * (double)(b > 1 ? b - 1 : 0); }
  // (:1728-1753) the k in 0..avail maximising expected tokens per unit cost, gain(k) =
  // 1 + p + ... + p^k over cost(k + 1); k = 0 unless strictly better. Every 24th "none"
  // retries min(avail, 2) so a source is measured again.
  int best_len(int c, int avail) {
    if (fixed || avail == 0) return avail;
    const double p = rate(c);
    double best_rate = 1.0 / cost(1), gain = 1.0, pk = 1.0;
    int best = 0;
    for (int k = 1; k <= avail; k++) {
      pk *= p;
      gain += pk;
      const double r = gain / cost(k + 1);
      if (r > best_rate) { best_rate = r; best = k; }
    }
    if (best == 0 && ++since_try >= 24) { since_try = 0; return std::min(avail, 2); }
    return best;
  }
  // (:1756-1760) forgets the accept rates, keeps the pass costs
  void reset_rates() {
    for (int i = 0; i < 4; i++) acc[i] = fail_[i] = 1.0;
    since_try = 0;
  }
  // (:1763-1774) decay 0.97 with a floor of 0.5 on every class, then count this verify
  void record_draft(int c, int drafted, int accepted) {
    for (int i = 0; i < 4; i++) { acc[i] = std::max(acc[i] * 0.97, 0.5); fail_[i] = std::max(fail_[i] * 0.97, 0.5); }
    acc[c] += accepted;
    if (accepted < drafted) fail_[c] += 1.0;
  }
  // (:1777-1785) whole microseconds, as the reference's u64
  void record_step(uint64_t us_i) {
    const double us = (double)us_i;
    t1_us = have_t1 ? 0.9 * t1_us + 0.1 * us : us;
    if (!have_extra) extra_us = 0.3 * t1_us;
    have_t1 = true;
  }
  // (:1788-1798) per-extra-row cost of a b-row verify, clamped to [0, 1.5 t1] before the average
  void record_verify(int b, uint64_t us_i) {
    if (b < 2 || !have_t1) return;
    const double m = std::min(std::max(((double)us_i - t1_us) / (double)(b - 1), 0.0), 1.5 * t1_us);
    extra_us = have_extra ? 0.85 * extra_us + 0.15 * m : m;
    have_extra = true;
  }
};

}  // namespace spx
