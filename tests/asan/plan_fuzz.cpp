// Planner fuzz driver for a sanitizer build (AddressSanitizer and
// UndefinedBehaviorSanitizer, g++ on the host): random ticks of decode and
// prefill sequences through hy_plan_tick, first with roomy buffers, then
// with buffers of exactly the counts it reported (guarded by poisoned
// margins the planner must not touch), then one record short of each
// (HY_ENOSPACE expected, nothing written past the end). Every plan is
// checked for coverage: each decode sequence's tokens once across its
// pieces, one merge item per decode sequence over its pieces' slots, each
// prefill tile's key range [0, cache + q1) once across its parts.
// Usage: plan_fuzz <seed> <ticks>; prints "ok <ticks>" and exits 0.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <random>
#include <vector>

#include "../../include/hayate_attn.h"
#include "../../hayate-exp_amd/csrc/decode_shape.h"
#include "../../hayate-exp_amd/csrc/prefill_shape.h"

namespace hy {
void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  va_end(ap);
}
void clear_error() {}
}  // namespace hy

namespace {

constexpr int32_t kPoison = 0x5a5a5a5a;
constexpr int kMargin = 64;  // int32 guard words after every buffer

#define CHECK(cond, ...)                                             \
  do {                                                               \
    if (!(cond)) {                                                   \
      fprintf(stderr, "check failed (%s:%d): %s\n", __FILE__, __LINE__, #cond); \
      fprintf(stderr, __VA_ARGS__);                                  \
      fprintf(stderr, "\n");                                         \
      exit(1);                                                       \
    }                                                                \
  } while (0)

struct Buffers {
  std::vector<int32_t> dec, mrg, pre, pmrg;
  int32_t counts[7];
  void size(int dec_cap, int mrg_cap, int pre_cap, int pmrg_cap) {
    dec.assign(8 * static_cast<size_t>(dec_cap) + kMargin, kPoison);
    mrg.assign(4 * static_cast<size_t>(mrg_cap) + kMargin, kPoison);
    pre.assign(8 * static_cast<size_t>(pre_cap) + kMargin, kPoison);
    pmrg.assign(8 * static_cast<size_t>(pmrg_cap) + kMargin, kPoison);
  }
  bool guards_intact(int dec_cap, int mrg_cap, int pre_cap, int pmrg_cap) const {
    auto intact = [](const std::vector<int32_t> &v, size_t used) {
      for (size_t i = used; i < v.size(); ++i)
        if (v[i] != kPoison) return false;
      return true;
    };
    return intact(dec, 8 * static_cast<size_t>(dec_cap)) &&
           intact(mrg, 4 * static_cast<size_t>(mrg_cap)) &&
           intact(pre, 8 * static_cast<size_t>(pre_cap)) &&
           intact(pmrg, 8 * static_cast<size_t>(pmrg_cap));
  }
};

int plan(const std::vector<int32_t> &q, const std::vector<int32_t> &kv, int hq, int hkv,
         int page, int cus, int split, Buffers &b, int dec_cap, int mrg_cap, int pre_cap,
         int pmrg_cap) {
  b.size(dec_cap, mrg_cap, pre_cap, pmrg_cap);
  const int rc = hy_plan_tick(q.data(), kv.data(), static_cast<int32_t>(q.size()), hq, hkv,
                              page, cus, split, b.dec.data(), dec_cap, b.mrg.data(), mrg_cap,
                              b.pre.data(), pre_cap, b.pmrg.data(), pmrg_cap, b.counts);
  CHECK(b.guards_intact(dec_cap, mrg_cap, pre_cap, pmrg_cap), "write past a buffer (rc %d)", rc);
  return rc;
}

void check_plan(const std::vector<int32_t> &q, const std::vector<int32_t> &kv, int G,
                const Buffers &b) {
  const int nc = b.counts[0], nm = b.counts[1], npf = b.counts[3], npm = b.counts[4];
  const int np = b.counts[6];
  const int n = static_cast<int>(q.size());
  // decode: pieces of each sequence are consecutive and tile [0, kv)
  std::vector<int64_t> covered(n, 0);
  std::vector<int> first_piece(n, -1), pieces_of(n, 0);
  const int32_t *pieces = b.dec.data() + 8 * nc;
  for (int c = 0; c < nc; ++c) {
    const int32_t *ch = b.dec.data() + 8 * c;
    CHECK(ch[0] < ch[1] && ch[1] <= np, "chunk %d pieces [%d, %d) of %d", c, ch[0], ch[1], np);
    CHECK(c == 0 || ch[0] == b.dec[8 * (c - 1) + 1], "chunk %d not contiguous", c);
  }
  for (int p = 0; p < np; ++p) {
    const int32_t *pr = pieces + 8 * p;
    const int s = pr[0];
    CHECK(s >= 0 && s < n && q[s] == 1, "piece %d of sequence %d", p, s);
    CHECK(pr[1] == covered[s] && pr[2] > pr[1] && pr[2] <= kv[s], "piece %d range", p);
    covered[s] = pr[2];
    if (first_piece[s] < 0) first_piece[s] = p;
    CHECK(first_piece[s] + pieces_of[s] == p, "pieces of sequence %d not consecutive", s);
    ++pieces_of[s];
  }
  int n_dec = 0;
  for (int s = 0; s < n; ++s)
    if (q[s] == 1) {
      CHECK(covered[s] == kv[s], "sequence %d covered %lld of %d", s,
            static_cast<long long>(covered[s]), kv[s]);
      ++n_dec;
    }
  CHECK(nm == n_dec, "%d merge items for %d decode sequences", nm, n_dec);
  for (int m = 0; m < nm; ++m) {
    const int32_t *it = b.mrg.data() + 4 * m;
    const int s = it[0];
    CHECK(s >= 0 && s < n && q[s] == 1, "merge item %d", m);
    CHECK(it[1] == pieces[8 * first_piece[s] + 3], "merge item %d first slot", m);
    CHECK(it[2] == hy::kDecodeWaves * pieces_of[s], "merge item %d partials", m);
  }
  // prefill: each tile's parts partition [0, cache + q1)
  const int tile = hy::kPrefillRows / G;
  std::vector<std::vector<std::pair<int, int>>> parts(n);
  for (int i = 0; i < npf; ++i) {
    const int32_t *it = b.pre.data() + 8 * i;
    const int s = it[0];
    CHECK(s >= 0 && s < n && q[s] > 1, "prefill item %d of sequence %d", i, s);
    CHECK(it[1] % tile == 0 && it[2] == std::min(q[s], it[1] + tile), "prefill item %d tile", i);
    CHECK(it[3] < it[4], "prefill item %d keys", i);
    parts[s].push_back({it[1] * 65536 + it[3], it[4]});
  }
  for (int s = 0; s < n; ++s) {
    if (q[s] <= 1) continue;
    std::sort(parts[s].begin(), parts[s].end());
    const int cache = kv[s] - q[s];
    size_t k = 0;
    for (int q0 = 0; q0 < q[s]; q0 += tile) {
      const int q1 = std::min(q[s], q0 + tile);
      int at = 0;
      while (k < parts[s].size() && parts[s][k].first / 65536 == q0) {
        CHECK(parts[s][k].first % 65536 == at, "sequence %d tile %d gap at key %d", s, q0, at);
        at = parts[s][k].second;
        ++k;
      }
      CHECK(at == cache + q1, "sequence %d tile %d keys end at %d, not %d", s, q0, at, cache + q1);
    }
    CHECK(k == parts[s].size(), "sequence %d: extra prefill parts", s);
  }
  CHECK(npm <= npf, "%d prefill merges for %d items", npm, npf);
}

}  // namespace

int main(int argc, char **argv) {
  const unsigned seed = argc > 1 ? static_cast<unsigned>(atoi(argv[1])) : 1;
  const int ticks = argc > 2 ? atoi(argv[2]) : 200;
  std::mt19937 rng(seed);
  auto uni = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
  const int groups[] = {1, 2, 4, 8, 16};
  for (int t = 0; t < ticks; ++t) {
    const int hkv = uni(1, 8);
    const int G = groups[uni(0, 4)];
    const int page = 32 << uni(0, 3);
    const int cus = uni(0, 3) == 0 ? 0 : uni(1, 304);
    const int split = uni(0, 4) == 0 ? uni(32, 2048) : 0;
    const int n = uni(0, 70);
    std::vector<int32_t> q(n), kv(n);
    for (int s = 0; s < n; ++s) {
      const int kind = uni(0, 9);
      q[s] = kind < 6 ? 1 : (kind < 8 ? uni(2, 1100) : uni(0, 1));
      const int depth = uni(0, 3) == 0 ? uni(0, 40000) : uni(0, 3000);
      kv[s] = q[s] + (q[s] == 0 ? 0 : depth);
    }
    // roomy buffers first: the counts say what a tight run needs
    Buffers roomy;
    const int big = 40000;
    int rc = plan(q, kv, G * hkv, hkv, page, cus, split, roomy, big, n + 1, big, big);
    CHECK(rc == HY_OK, "tick %d: rc %d", t, rc);
    check_plan(q, kv, G, roomy);
    const int nd = roomy.counts[0] + roomy.counts[6], nm = roomy.counts[1];
    const int npf = roomy.counts[3], npm = roomy.counts[4];
    Buffers tight;
    rc = plan(q, kv, G * hkv, hkv, page, cus, split, tight, nd, nm, npf, npm);
    CHECK(rc == HY_OK, "tick %d: exact capacities refused (rc %d)", t, rc);
    check_plan(q, kv, G, tight);
    for (int which = 0; which < 4; ++which) {
      int caps[4] = {nd, nm, npf, npm};
      if (caps[which] == 0) continue;
      --caps[which];
      Buffers shortb;
      rc = plan(q, kv, G * hkv, hkv, page, cus, split, shortb, caps[0], caps[1], caps[2],
                caps[3]);
      CHECK(rc == HY_ENOSPACE, "tick %d: capacity %d one short gave rc %d", t, which, rc);
    }
  }
  printf("ok %d\n", ticks);
  return 0;
}
