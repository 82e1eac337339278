// viterbi.cpp — host-side BIOES Viterbi decode of the forward's logits.
//
// Restates ViterbiDecoder (packages/textsift/src/browser/inference/viterbi.ts)
// with the reference's arithmetic: the score tables and the alpha lattice are
// f32 arrays (Float32Array), every sum is formed in double (a JS number) and
// rounded to f32 when stored, comparisons are strict (the first maximum
// wins), and the running best starts at the double -1e30 with predecessor 0.
// Sequences of a batch are decoded on separate host threads.
#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "pfhip_internal.h"

namespace pf {
namespace {

constexpr int kClasses = 33;   // NUM_BIOES_CLASSES (viterbi.ts:37)
constexpr int kLabels = 8;     // NUM_SPAN_LABELS (viterbi.ts:38)
constexpr float kNegInfF = -1e30f;
constexpr double kNegInf = -1e30;

inline int tag_of(int label, int boundary) { return 1 + label * 4 + boundary; }  // bioesTagOf (viterbi.ts:47-49)

// buildTransitionMatrix (viterbi.ts:159-206): trans[to * C + from].
// bias order: backgroundStay, backgroundToStart, insideToContinue,
// insideToEnd, endToBackground, endToStart (model/calibration.ts:29-36).
void build_tables(const float* bias, float* trans, float* start) {
  std::fill(trans, trans + kClasses * kClasses, kNegInfF);
  auto allow = [&](int from, int to, float s) { trans[to * kClasses + from] = s; };
  allow(0, 0, bias[0]);
  for (int l = 0; l < kLabels; ++l) {
    const int B = tag_of(l, 0), I = tag_of(l, 1), E = tag_of(l, 2), S = tag_of(l, 3);
    allow(0, B, bias[1]);
    allow(0, S, bias[1]);
    allow(B, I, bias[2]);
    allow(B, E, bias[3]);
    allow(I, I, bias[2]);
    allow(I, E, bias[3]);
    allow(E, 0, bias[4]);
    allow(S, 0, bias[4]);
    for (int l2 = 0; l2 < kLabels; ++l2) {
      const int B2 = tag_of(l2, 0), S2 = tag_of(l2, 3);
      allow(E, B2, bias[5]);
      allow(E, S2, bias[5]);
      allow(S, B2, bias[5]);
      allow(S, S2, bias[5]);
    }
  }
  // buildStartScores (viterbi.ts:208-218): O, B-*, S-* may start a sequence
  std::fill(start, start + kClasses, kNegInfF);
  start[0] = 0.0f;
  for (int l = 0; l < kLabels; ++l) start[tag_of(l, 0)] = start[tag_of(l, 3)] = 0.0f;
}

// ViterbiDecoder.decode (viterbi.ts:85-146) for one sequence of T tokens.
void decode_one(const float* logits, int T, const float* trans, const float* start, uint8_t* tags) {
  if (T <= 0) return;
  const int C = kClasses;
  std::vector<float> alpha((size_t)T * C);
  std::vector<uint8_t> back((size_t)T * C);
  for (int j = 0; j < C; ++j) {
    alpha[j] = (float)((double)start[j] + (double)logits[j]);
    back[j] = 0xFF;
  }
  for (int t = 1; t < T; ++t) {
    const float* prev = alpha.data() + (size_t)(t - 1) * C;
    float* cur = alpha.data() + (size_t)t * C;
    const float* em = logits + (size_t)t * C;
    for (int j = 0; j < C; ++j) {
      const float* col = trans + j * C;
      double best = kNegInf;
      int arg = 0;
      for (int i = 0; i < C; ++i) {
        const double s = (double)prev[i] + (double)col[i];
        if (s > best) {
          best = s;
          arg = i;
        }
      }
      cur[j] = (float)(best + (double)em[j]);
      back[(size_t)t * C + j] = (uint8_t)arg;
    }
  }
  const float* last = alpha.data() + (size_t)(T - 1) * C;
  double best = kNegInf;
  int fin = 0;
  for (int j = 0; j < C; ++j)
    if ((double)last[j] > best) {
      best = last[j];
      fin = j;
    }
  tags[T - 1] = (uint8_t)fin;
  for (int t = T - 1; t > 0; --t) tags[t - 1] = back[(size_t)t * C + tags[t]];
}

}  // namespace
}  // namespace pf

extern "C" int pfhip_viterbi_decode(const float* logits, uint32_t batch, uint32_t seq_stride,
                                    const uint32_t* seq_lens, uint32_t num_classes, const float* biases,
                                    uint8_t* tags, uint32_t n_threads, char* err, size_t err_cap) {
  try {
    PF_CHECK(num_classes == (uint32_t)pf::kClasses,
             "viterbi_decode: expected 33 classes, got " + std::to_string(num_classes));
    PF_CHECK(batch == 0 || (logits && biases && tags), "viterbi_decode: null argument");
    for (uint32_t b = 0; b < batch; ++b)
      if (seq_lens)
        PF_CHECK(seq_lens[b] <= seq_stride, "viterbi_decode: sequenceLength " + std::to_string(seq_lens[b]) +
                                                " exceeds logits.sequenceLength " + std::to_string(seq_stride));
    float trans[pf::kClasses * pf::kClasses], start[pf::kClasses];
    pf::build_tables(biases, trans, start);
    auto run = [&](uint32_t b) {
      const uint32_t T = seq_lens ? seq_lens[b] : seq_stride;
      pf::decode_one(logits + (size_t)b * seq_stride * pf::kClasses, (int)T, trans, start,
                     tags + (size_t)b * seq_stride);
    };
    uint32_t nt = n_threads ? n_threads : std::max(1u, std::thread::hardware_concurrency());
    nt = std::min(nt, batch);
    if (nt <= 1) {
      for (uint32_t b = 0; b < batch; ++b) run(b);
    } else {
      std::vector<std::thread> pool;
      for (uint32_t w = 0; w < nt; ++w)
        pool.emplace_back([&, w] {
          for (uint32_t b = w; b < batch; b += nt) run(b);
        });
      for (auto& th : pool) th.join();
    }
    return 0;
  } catch (const std::exception& ex) {
    pf::set_err(err, err_cap, ex.what());
    return -1;
  }
}
