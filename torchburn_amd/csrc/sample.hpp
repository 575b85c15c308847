// Internal launchers of the device sampler (sample.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tb {

struct DecState;

constexpr int kSampleSlice = 2048;     // logits per top-k block
constexpr int kSampleMaxK = 1024;      // largest top_k of the list / select path
constexpr int kSampleMaxBlocks = 128;  // vocabularies up to 262144
constexpr int kSampleLists = 4 * kSampleMaxBlocks;   // one per wave of the list kernel
constexpr int kSampleCand = kSampleLists * 8 * 2;     // u32 words of the wave lists

// Device-resident sampling parameters.  k: candidates (1 for greedy);
// greedy: take the top-1 of the raw logits; counter advances once per draw.
struct SampleParams {
    float temperature;
    float top_p;
    float penalty;
    int k;
    int greedy;
    int pad;
    unsigned long long seed;
    unsigned long long counter;
};

struct SampleOut {
    int token;   // the drawn token
    int kept;    // candidates after top-k
    float u;     // the uniform used (-1 when none was drawn)
    int pad;
};

// The repetition-penalty window of a generation loop: the last kSampleWindow
// tokens (decoder.rs:859-876), on the device, as a ring: the n live tokens
// sit in slots head, head + 1, ... (mod kSampleWindow).  The penalty only needs
// the set, so a push writes one slot instead of shifting the window.
constexpr int kSampleWindow = 64;
struct SampleWindow {
    int n;
    int head;
    int64_t tok[kSampleWindow];
};

// Device scratch of the sampler: key, idx and p each hold
// sample_scratch_items(V) entries, cnt kSampleLists.  k <= kSampleMaxK: key
// holds the wave lists (64-bit items, kSampleLists x 8) and cnt their wave
// counts; k > kSampleMaxK: the k items and their weights.
struct SampleScratch {
    uint32_t *key;
    int *idx;
    float *p;
    int *cnt;
};

inline int64_t sample_scratch_items(int64_t V) { return V > kSampleCand ? V : kSampleCand; }

int sample_blocks(int V);

// u of draw number `counter` under `seed` (the device's generator, on the host).
float sample_uniform(uint64_t seed, uint64_t counter);

// Penalty over `recent` (device int64, n_recent of them; logits modified in
// place), then top-k / temperature / top-p / draw per *prm into *out.
// large: the path for k > kSampleMaxK (prm->k must be on the same side; each
// path's kernels return at once for the other's k).
// Decoder form: with `win`, the step's input token (dstate->token) is pushed
// onto the window and the penalty covers the window; with `dstate`, the drawn
// token becomes the next step's input (history, token, pos, step), as the
// greedy argmax tail does.  Capturable in a graph.
int launch_sample(float *logits, int V, const int64_t *recent, int n_recent, SampleParams *prm,
                  const SampleScratch &ws, SampleOut *out, hipStream_t st, bool large,
                  SampleWindow *win = nullptr, DecState *dstate = nullptr,
                  int *history = nullptr, int hist_cap = 0);

}  // namespace tb
