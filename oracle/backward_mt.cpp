// backward_mt.cpp -- TEST INFRASTRUCTURE ONLY.  A multithreaded C++
// restatement of the TBE backward with exact rowwise Adagrad, used as the
// CPU baseline of the backward (bench.py's cpu_baseline leg) and checked
// bit for bit against the single-threaded restatement in mx_oracle.c
// (orc_backward_rowwise_adagrad, whose rule and citations it follows).
// Nothing in the product links, loads or calls this file.
//
// The work splits over key ranges, which is how the rows split: a run (the
// occurrences of one linearized key t-offset + row) updates one row, and
// distinct keys are distinct rows, so threads that own disjoint key ranges
// never touch the same weights or momentum.  Within a run the gradient slices
// are summed in position order, exactly as the single-threaded restatement
// does after its stable sort, so every result is identical to it.
//
//   1. linearize (threads over bag ranges): key[l] = hash_size_cumsum[t] +
//      indices[l], bag[l] = t*B + b;
//   2. split the key space into parts of about equal occurrence counts (a
//      coarse key histogram, summed over threads);
//   3. scatter each position into its part, positions ascending within a part
//      (per-thread counts over contiguous position ranges, then offsets);
//   4. threads take parts from a shared counter: sort the part's (key,
//      position) pairs, then for each run sum its slices in position order and
//      apply the update.
//
// Built with -ffp-contract=off: every product is rounded on its own, as in
// mx_oracle.c; std::fma is deliberate.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

template <class F>
void parallel_for(int nthreads, F f) {
  std::vector<std::thread> th;
  th.reserve(nthreads > 1 ? nthreads - 1 : 0);
  for (int i = 1; i < nthreads; ++i) th.emplace_back(f, i);
  f(0);
  for (auto& t : th) t.join();
}

}  // namespace

extern "C" int orc_backward_rowwise_adagrad_mt(
    float* W, const int64_t* w_off, const int32_t* D_off, int32_t T, int64_t B,
    const int64_t* hsc, int32_t bits, const int64_t* indices, const int64_t* offsets, int64_t N,
    int32_t pooling, const float* iw, const float* grad, int64_t total_D, float* m1,
    const int64_t* m1_off, float lr, float eps, float wd, int32_t wd_mode, int32_t nthreads) {
  if (N <= 0) return 0;
  if (nthreads < 1) nthreads = 1;
  const int64_t nbags = static_cast<int64_t>(T) * B;
  std::vector<int64_t> key(N);
  std::vector<int32_t> bag(N);
  std::atomic<int> bad{0};
  const uint64_t mask = bits >= 64 ? ~0ull : ((1ull << bits) - 1ull);
  // 1. linearize
  parallel_for(nthreads, [&](int i) {
    const int64_t b0 = nbags * i / nthreads, b1 = nbags * (i + 1) / nthreads;
    for (int64_t bg = b0; bg < b1; ++bg) {
      const int64_t t = bg / B;
      for (int64_t l = offsets[bg]; l < offsets[bg + 1]; ++l) {
        key[l] = hsc[t] + indices[l];
        bag[l] = static_cast<int32_t>(bg);
        // The sort orders keys by their low `bits` bits; keys above them
        // would order differently (the single-threaded restatement covers that).
        if (key[l] < 0 || (static_cast<uint64_t>(key[l]) & ~mask) != 0) bad.store(1);
      }
    }
  });
  if (bad.load()) return -3;
  // 2. parts of about equal occurrence counts over a coarse key histogram
  const int64_t kmax = hsc[T] > 1 ? hsc[T] : 1;
  int shift = 0;
  while ((kmax >> shift) > (1 << 16)) ++shift;
  const int64_t nbuck = (kmax >> shift) + 1;
  std::vector<std::vector<int64_t>> th_hist(nthreads, std::vector<int64_t>(nbuck, 0));
  parallel_for(nthreads, [&](int i) {
    const int64_t l0 = N * i / nthreads, l1 = N * (i + 1) / nthreads;
    auto& h = th_hist[i];
    for (int64_t l = l0; l < l1; ++l) {
      const int64_t k = key[l] >> shift;
      ++h[k < nbuck ? k : nbuck - 1];
    }
  });
  std::vector<int64_t> hist(nbuck, 0);
  for (auto& h : th_hist)
    for (int64_t k = 0; k < nbuck; ++k) hist[k] += h[k];
  const int64_t want_parts = static_cast<int64_t>(nthreads) * 16;
  std::vector<int32_t> part_of(nbuck);
  int32_t nparts = 0;
  {
    int64_t acc = 0;
    const int64_t per = (N + want_parts - 1) / want_parts;
    for (int64_t k = 0; k < nbuck; ++k) {
      part_of[k] = nparts;
      acc += hist[k];
      if (acc >= per) {
        ++nparts;
        acc = 0;
      }
    }
    if (acc > 0 || nparts == 0) ++nparts;
    for (auto& p : part_of) p = std::min(p, nparts - 1);
  }
  // 3. scatter positions into parts, ascending within a part
  std::vector<std::vector<int64_t>> cnt(nthreads, std::vector<int64_t>(nparts, 0));
  parallel_for(nthreads, [&](int i) {
    const int64_t l0 = N * i / nthreads, l1 = N * (i + 1) / nthreads;
    for (int64_t l = l0; l < l1; ++l) {
      const int64_t k = std::min(key[l] >> shift, nbuck - 1);
      ++cnt[i][part_of[k]];
    }
  });
  std::vector<int64_t> part_start(nparts + 1, 0);
  {
    int64_t acc = 0;
    for (int32_t p = 0; p < nparts; ++p) {
      part_start[p] = acc;
      for (int i = 0; i < nthreads; ++i) {
        const int64_t c = cnt[i][p];
        cnt[i][p] = acc;  // thread i's first slot in part p
        acc += c;
      }
    }
    part_start[nparts] = acc;
  }
  std::vector<int64_t> pos(N);
  parallel_for(nthreads, [&](int i) {
    const int64_t l0 = N * i / nthreads, l1 = N * (i + 1) / nthreads;
    auto& slot = cnt[i];
    for (int64_t l = l0; l < l1; ++l) {
      const int64_t k = std::min(key[l] >> shift, nbuck - 1);
      pos[slot[part_of[k]]++] = l;
    }
  });
  // 4. parts: sort by (key, position), then runs
  std::atomic<int32_t> next{0};
  const bool mean = pooling == 1;
  parallel_for(nthreads, [&](int) {
    std::vector<uint64_t> order;
    std::vector<float> g(1024);
    for (int32_t p = next.fetch_add(1); p < nparts; p = next.fetch_add(1)) {
      const int64_t s = part_start[p], e = part_start[p + 1];
      if (s == e) continue;
      int64_t klo = key[pos[s]];
      for (int64_t j = s; j < e; ++j) klo = std::min(klo, key[pos[j]]);
      order.resize(e - s);
      for (int64_t j = s; j < e; ++j)
        order[j - s] = (static_cast<uint64_t>(key[pos[j]] - klo) << 32) |
                       static_cast<uint64_t>(j - s);
      std::sort(order.begin(), order.end());  // positions ascend within a part: stable
      for (size_t a = 0; a < order.size();) {
        const uint64_t kk = order[a] >> 32;
        size_t b = a;
        while (b < order.size() && (order[b] >> 32) == kk) ++b;
        // run [a, b): the row of the first occurrence's table
        const int64_t l0 = pos[s + static_cast<int64_t>(order[a] & 0xffffffffu)];
        const int64_t t = bag[l0] / B;
        const int32_t D = D_off[t + 1] - D_off[t];
        if (D > 1024) {
          bad.store(1);
          return;
        }
        const int64_t idx = key[l0] - hsc[t];
        for (int32_t d = 0; d < D; ++d) g[d] = 0.0f;
        for (size_t j = a; j < b; ++j) {
          const int64_t l = pos[s + static_cast<int64_t>(order[j] & 0xffffffffu)];
          const int64_t bg = bag[l];
          const int64_t tj = bg / B, bj = bg % B;
          if (D_off[tj + 1] - D_off[tj] != D) {  // one key, two widths: not one table
            bad.store(1);
            return;
          }
          const float* gr = grad + bj * total_D + D_off[tj];
          const int64_t L = offsets[bg + 1] - offsets[bg];
          const float sc = mean ? 1.0f / static_cast<float>(L) : 1.0f;  // L >= 1 here
          const float wl = iw ? iw[l] : 1.0f;
          for (int32_t d = 0; d < D; ++d) g[d] = g[d] + (gr[d] * sc) * wl;
        }
        float* w = W + w_off[t] + idx * D;
        float ss = 0.0f;
        for (int32_t d = 0; d < D; ++d) {
          const float sd = wd_mode == 1 ? std::fma(wd, w[d], g[d]) : g[d];
          ss = ss + sd * sd;
        }
        float* h = m1 + m1_off[t] + idx;
        const float hn = *h + ss / static_cast<float>(D);
        const float m = lr / (std::sqrt(hn) + eps);
        float c = 1.0f;
        if (wd_mode == 1) c = 1.0f - m * wd;
        if (wd_mode == 2) c = 1.0f - lr * wd;
        for (int32_t d = 0; d < D; ++d) w[d] = std::fma(-m, g[d], c * w[d]);
        *h = hn;
        a = b;
      }
    }
  });
  return bad.load() ? -1 : 0;
}
