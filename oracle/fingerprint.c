/* C restatement of recompute.fingerprint's three sums (oracle: test infrastructure only).
 *
 * recompute.py:59-61 (constants) and :93-116 (_lsr, _fp_weights, _fingerprint_torch): for signed words b at
 * positions p,  z = p + SEED; z = (z ^ z>>30) * M1; z = (z ^ z>>27) * M2; z ^= z>>31  (logical shifts on
 * uint64), w1 = z | 1, w2 = (z ^ z>>32) | 1, sums (b, b*w1, b*w2) mod 2^64.
 * Used to time the CPU baseline and to check the numpy version on large inputs. */
#include <stdint.h>
#include <pthread.h>

#define FP_SEED 0x9E3779B97F4A7C15ULL
#define FP_M1 0xBF58476D1CE4E5B9ULL
#define FP_M2 0x94D049BB133111EBULL

static inline void weights(uint64_t p, uint64_t *w1, uint64_t *w2) {
  uint64_t z = p + FP_SEED;
  z = (z ^ (z >> 30)) * FP_M1;
  z = (z ^ (z >> 27)) * FP_M2;
  z ^= z >> 31;
  *w1 = z | 1;
  *w2 = (z ^ (z >> 32)) | 1;
}

void oracle_fp3_i16(const int16_t *b, int64_t n, int64_t start, int64_t *out) {
  uint64_t s0 = 0, s1 = 0, s2 = 0;
  for (int64_t i = 0; i < n; ++i) {
    uint64_t w1, w2, v = (uint64_t)(int64_t)b[i];
    weights((uint64_t)(start + i), &w1, &w2);
    s0 += v; s1 += v * w1; s2 += v * w2;
  }
  out[0] = (int64_t)s0; out[1] = (int64_t)s1; out[2] = (int64_t)s2;
}

void oracle_fp3_i8(const int8_t *b, int64_t n, int64_t start, int64_t *out) {
  uint64_t s0 = 0, s1 = 0, s2 = 0;
  for (int64_t i = 0; i < n; ++i) {
    uint64_t w1, w2, v = (uint64_t)(int64_t)b[i];
    weights((uint64_t)(start + i), &w1, &w2);
    s0 += v; s1 += v * w1; s2 += v * w2;
  }
  out[0] = (int64_t)s0; out[1] = (int64_t)s1; out[2] = (int64_t)s2;
}

struct kv_job { const int16_t *b; int64_t nblk, words, lo, hi; int64_t *out; };

static void *kv_run(void *arg) {
  struct kv_job *j = (struct kv_job *)arg;
  for (int64_t blk = j->lo; blk < j->hi; ++blk)
    oracle_fp3_i16(j->b + blk * j->words, j->words, 0, j->out + 3 * blk);
  return 0;
}

/* every block of a paged cache: blocks of `words` int16 words each, positions numbered from 0 per block */
void oracle_kv_fp3_i16(const int16_t *b, int64_t nblk, int64_t words, int64_t *out, int threads) {
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  pthread_t tid[64];
  struct kv_job jobs[64];
  int64_t per = (nblk + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    int64_t lo = t * per, hi = lo + per < nblk ? lo + per : nblk;
    jobs[t] = (struct kv_job){b, nblk, words, lo < nblk ? lo : nblk, hi, out};
    pthread_create(&tid[t], 0, kv_run, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(tid[t], 0);
}
