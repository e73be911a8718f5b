// Host emulation of the wavefront top-k (larder_amd/csrc/lmoe_common.h, topk_wave): 64 lanes as loops, a ballot
// as a 64-bit mask, the LDS pick area as an array of 64 words. Two threshold searches: the kernel's, one bit a
// step (up to 32 steps, stopping once exactly k keys are at or above the prefix), and a two-bits-a-step form (16
// steps, three candidates a step). A third form emulates rank_pick_wave (the pick of one rank, no compaction). Used by
// tests/test_topk_emulation.py to check, on the CPU, that both give the oracle's picks on tie-heavy rows and that
// the compaction never writes more than k picks.
//
// stdin: "rows E k" then rows lines of E float32 bit patterns (hex); stdout per row: "ok|BAD n_picks ids..." for
// each search, then "ok k ids..." of rank_pick_wave for ranks 0 .. k - 1. argv[1]: a slip planted in a search (0:
// none; 1-3 the two-bit one, 4 the one-bit one, 5-6 rank_pick).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

static uint32_t logit_key(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if (f == 0.0f) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static int popc(uint64_t m) { return __builtin_popcountll(m); }

static int g_slip = 0;

// the k-th largest key: bit b stays set when at least k keys are >= the prefix; the search stops at a prefix with
// exactly k keys at or above it (the same picks). slip 4 (planted on the CPU only): it stops at the first prefix with
// at least k, a threshold too low whenever more than k keys are above it
static uint32_t thr_one_bit(const std::vector<uint32_t> &key, int k) {
  uint32_t thr = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = thr | (1u << b);
    int cnt = 0;
    for (uint32_t v : key) cnt += v >= cand;
    if (cnt >= k) {
      thr = cand;
      if (cnt == k || g_slip == 4) break;
    }
  }
  return thr;
}

// two bits a step: the three candidates prefix | 01, 10, 11 at bits (b, b - 1), the largest with >= k keys above it.
// slip (planted on the CPU only, to show the check has teeth): 1 = a candidate kept when more than k keys are above
// it (> for >=); 2 = the candidates tried low to high, the first with enough keys kept; 3 = the loop stopping one
// step early (b > 1), so the threshold's two lowest bits stay clear
static uint32_t thr_two_bit(const std::vector<uint32_t> &key, int k) {
  uint32_t thr = 0;
  for (int b = 31; g_slip == 3 ? b > 1 : b >= 1; b -= 2) {
    int cnt[4] = {0, 0, 0, 0};
    for (int c = 1; c < 4; ++c) {
      const uint32_t cand = thr | (uint32_t(c) << (b - 1));
      for (uint32_t v : key) cnt[c] += v >= cand;
    }
    int c;
    if (g_slip == 1)
      c = cnt[3] > k ? 3 : cnt[2] > k ? 2 : cnt[1] > k ? 1 : 0;
    else if (g_slip == 2)
      c = cnt[1] >= k ? 1 : cnt[2] >= k ? 2 : cnt[3] >= k ? 3 : 0;
    else
      c = cnt[3] >= k ? 3 : cnt[2] >= k ? 2 : cnt[1] >= k ? 1 : 0;
    thr |= uint32_t(c) << (b - 1);
  }
  return thr;
}

// steps 2 and 3 of topk_wave for one token: keys key[lane + 64 j] (0 past E), the picks compacted in index order
// into lds[0..31] / lds[32..63] (a write at pos >= 32 is counted as an overrun, not made), then ranked
static int picks(const std::vector<uint32_t> &key, int E, int k, uint32_t thr, std::vector<uint32_t> &ids,
                 int *overrun) {
  const int NPL = (E + 63) / 64;
  uint32_t lds[64] = {0};
  int n_gt = 0;
  for (int j = 0; j < NPL; ++j) {
    uint64_t m = 0;
    for (int lane = 0; lane < 64; ++lane)
      if (key[lane + 64 * j] > thr) m |= uint64_t(1) << lane;
    n_gt += popc(m);
  }
  const int need = k - n_gt;
  int eq_before = 0, sel_before = 0, n_sel = 0;
  *overrun = 0;
  for (int j = 0; j < NPL; ++j) {
    uint64_t eq = 0, selm = 0;
    for (int lane = 0; lane < 64; ++lane)
      if (key[lane + 64 * j] == thr) eq |= uint64_t(1) << lane;
    bool sel[64];
    for (int lane = 0; lane < 64; ++lane) {
      const uint64_t below = (uint64_t(1) << lane) - 1;
      const uint32_t kv = key[lane + 64 * j];
      const bool tie = (eq >> lane) & 1u;
      sel[lane] = kv > thr || (tie && eq_before + popc(eq & below) < need);
      if (sel[lane]) selm |= uint64_t(1) << lane;
    }
    for (int lane = 0; lane < 64; ++lane) {
      if (!sel[lane]) continue;
      const int pos = sel_before + popc(selm & ((uint64_t(1) << lane) - 1));
      ++n_sel;
      if (pos >= 32) {
        ++*overrun;
        continue;
      }
      lds[pos] = key[lane + 64 * j];
      lds[32 + pos] = uint32_t(lane + 64 * j);
    }
    eq_before += popc(eq);
    sel_before += popc(selm);
  }
  ids.assign(k, 0xFFFFFFFFu);
  for (int lane = 0; lane < k && lane < 32; ++lane) {
    int rank = 0;
    for (int o = 0; o < k; ++o)
      rank += (lds[o] > lds[lane] || (lds[o] == lds[lane] && lds[32 + o] < lds[32 + lane])) ? 1 : 0;
    if (rank < k) ids[rank] = lds[32 + lane];
  }
  return n_sel;
}

// rank_pick_wave: the expert of rank `want` (larger logit first, equal logits by lower index) without the top-k's
// compaction and ranking. The one-bit search for the (want + 1)-th largest key; stopped at a prefix with exactly
// want + 1 keys at or above it, rank want is the smallest of those keys, the highest index among equal ones; run to
// the end, the prefix is that key itself and rank want is the (want + 1 - #keys above it)-th lowest index holding it.
// Slips (planted on the CPU only): 5 = the lowest index among the smallest keys in the stopped case; 6 = the keys
// above the threshold not subtracted in the full case.
static uint32_t rank_pick(const std::vector<uint32_t> &key, int want) {
  const int NPL = int(key.size()) / 64, need = want + 1;
  uint32_t thr = 0;
  bool exact = false;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = thr | (1u << b);
    int cnt = 0;
    for (uint32_t v : key) cnt += v >= cand;
    if (cnt >= need) {
      thr = cand;
      if (cnt == need) {
        exact = true;
        break;
      }
    }
  }
  if (exact) {
    uint32_t m = 0xFFFFFFFFu;
    for (uint32_t v : key)
      if (v >= thr && v < m) m = v;
    if (g_slip == 5) {
      for (int j = 0; j < NPL; ++j)
        for (int lane = 0; lane < 64; ++lane)
          if (key[lane + 64 * j] == m) return uint32_t(lane + 64 * j);
      return 0xFFFFFFFFu;
    }
    for (int j = NPL - 1; j >= 0; --j) {
      uint64_t eq = 0;
      for (int lane = 0; lane < 64; ++lane)
        if (key[lane + 64 * j] == m) eq |= uint64_t(1) << lane;
      if (eq) return uint32_t(64 * j + 63 - __builtin_clzll(eq));
    }
    return 0xFFFFFFFFu;
  }
  int n_gt = 0;
  for (uint32_t v : key) n_gt += v > thr;
  int rem = need - (g_slip == 6 ? 0 : n_gt);
  for (int j = 0; j < NPL; ++j) {
    uint64_t eq = 0;
    for (int lane = 0; lane < 64; ++lane)
      if (key[lane + 64 * j] == thr) eq |= uint64_t(1) << lane;
    const int c = popc(eq);
    if (rem <= c) {
      for (int i = 1; i < rem; ++i) eq &= eq - 1;
      return uint32_t(64 * j + __builtin_ctzll(eq));
    }
    rem -= c;
  }
  return 0xFFFFFFFFu;
}

int main(int argc, char **argv) {
  if (argc > 1) g_slip = std::atoi(argv[1]);
  int rows, E, k;
  if (std::scanf("%d %d %d", &rows, &E, &k) != 3) return 2;
  const int NPL = (E + 63) / 64;
  for (int r = 0; r < rows; ++r) {
    std::vector<uint32_t> key(64 * NPL, 0u);
    for (int e = 0; e < E; ++e) {
      unsigned bits;
      if (std::scanf("%x", &bits) != 1) return 2;
      float f;
      std::memcpy(&f, &bits, 4);
      key[e] = logit_key(f);
    }
    for (int form = 0; form < 2; ++form) {
      const uint32_t thr = form == 0 ? thr_one_bit(key, k) : thr_two_bit(key, k);
      std::vector<uint32_t> ids;
      int overrun = 0;
      const int n = picks(key, E, k, thr, ids, &overrun);
      std::printf("%s %d", (n == k && overrun == 0) ? "ok" : "BAD", n);
      for (uint32_t i : ids) std::printf(" %u", i);
      std::printf(" |");
    }
    // the third form: rank_pick for every rank of the top k
    std::printf(" ok %d", k);
    for (int w = 0; w < k; ++w) std::printf(" %u", rank_pick(key, w));
    std::printf("\n");
  }
  return 0;
}
