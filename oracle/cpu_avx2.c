/*
 * The CPU baseline: golem's x86 path for the quantised products -- its AVX2
 * kernels and its worker pool -- restated in C with intrinsics.
 *
 * TEST AND BENCHMARK INFRASTRUCTURE ONLY.  bench.py's cpu_baseline leg times
 * it on the GPU host's cores, and tests/ check it against the generic
 * restatement in oracle.c.  Nothing in golem_amd/ links or calls it.
 *
 * What is restated, and from where:
 *   - the worker pool: nn/parallel.go:36-191 (persistent workers as many as the
 *     threads allowed, spin 200,000 rounds of eight PAUSE then park, ranges
 *     handed out ceil(n / (4 chunks)) at a time, the caller takes ranges too,
 *     one section at a time), with the work threshold of nn/kernel.go:24;
 *   - dotQ6_KAVX2 (nn/dot_q6_k_amd64.s:62-125): the same integer steps, so the
 *     result is bit-identical to dotQ6_KGo (nn/dot_q6_k_test.go:51-75 holds
 *     golem to that), and matVecQ6_KRows' single-column loop
 *     (nn/dot_q6_k.go:77-103);
 *   - dotQ4_0AVX2 / x4 / x8 (nn/dot_q4_0_amd64.s:63-398) with their Begin /
 *     Finish state (nn/dot_q4_0.go:99-114), and matVecQ4_0Rows' tiling
 *     (nn/dot_q4_0.go:147-270): eight columns, then four, then one; stretches
 *     of 2048 inputs; row tiles of 24 KiB of weights, at most 64 rows.
 *
 * Build: gcc -O2 -mavx2 -mfma -mf16c -ffp-contract=off -pthread (oracle/build.py).
 */
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- the worker pool (nn/parallel.go) --------------------------------- */

#define SPIN_ROUNDS 200000           /* nn/parallel.go:38 */
#define PARALLEL_THRESHOLD (1 << 19) /* nn/kernel.go:24 */

typedef void (*cpu_work)(void *arg, int start, int end);

/* A worker's wake-up: a flag under a mutex, set at most once before it is
 * taken, like the one-slot channel a Go worker blocks on. */
struct slot {
    pthread_mutex_t mu;
    pthread_cond_t cv;
    int pending;
    atomic_int sleeping;
};

static struct {
    int count;
    cpu_work work;
    void *arg;
    int n, grain;
    atomic_long cursor;
    atomic_ulong sequence;
    atomic_long remaining;
    atomic_int spin;
    struct slot *slots;
    pthread_mutex_t section;
} pool = {.section = PTHREAD_MUTEX_INITIALIZER};

static pthread_mutex_t pool_init_mu = PTHREAD_MUTEX_INITIALIZER;

static void spin_pause(void) {
    for (int i = 0; i < 8; i++)
        _mm_pause();
}

static void consume(void) {
    for (;;) {
        const long start = atomic_fetch_add(&pool.cursor, pool.grain);
        if (start >= pool.n)
            return;
        const long end = start + pool.grain < pool.n ? start + pool.grain : pool.n;
        pool.work(pool.arg, (int)start, (int)end);
    }
}

static void park(struct slot *s) {
    pthread_mutex_lock(&s->mu);
    while (!s->pending)
        pthread_cond_wait(&s->cv, &s->mu);
    s->pending = 0;
    pthread_mutex_unlock(&s->mu);
}

static void wake(struct slot *s) {
    pthread_mutex_lock(&s->mu);
    s->pending = 1;
    pthread_cond_signal(&s->cv);
    pthread_mutex_unlock(&s->mu);
}

static void *serve(void *p) {
    struct slot *s = &pool.slots[(intptr_t)p];
    unsigned long last = 0;
    for (;;) {
        int spins = 0;
        while (atomic_load(&pool.sequence) == last) {
            spins++;
            if (spins > SPIN_ROUNDS || !atomic_load(&pool.spin)) {
                atomic_store(&s->sleeping, 1);
                /* a section published between the test and the flag */
                if (atomic_load(&pool.sequence) != last) {
                    atomic_store(&s->sleeping, 0);
                    break;
                }
                park(s);
                atomic_store(&s->sleeping, 0);
                spins = 0;
            }
            spin_pause();
        }
        last = atomic_load(&pool.sequence);
        consume();
        atomic_fetch_sub(&pool.remaining, 1);
    }
    return NULL;
}

/* Starts `threads` - 1 workers; the caller is the last one.  Once per process;
 * a later call with another count fails. */
int cpu_pool_init(int threads) {
    int rc = 0;
    pthread_mutex_lock(&pool_init_mu);
    if (pool.count) {
        rc = pool.count == threads ? 0 : -1;
    } else if (threads < 1) {
        rc = -2;
    } else {
        pool.slots = calloc((size_t)threads, sizeof(struct slot));
        for (int i = 0; i < threads; i++) {
            pthread_mutex_init(&pool.slots[i].mu, NULL);
            pthread_cond_init(&pool.slots[i].cv, NULL);
        }
        pool.count = threads;
        for (int i = 1; i < threads; i++) {
            pthread_t t;
            pthread_attr_t a;
            pthread_attr_init(&a);
            pthread_attr_setdetachstate(&a, PTHREAD_CREATE_DETACHED);
            if (pthread_create(&t, &a, serve, (void *)(intptr_t)i) != 0)
                rc = -3;
            pthread_attr_destroy(&a);
        }
    }
    pthread_mutex_unlock(&pool_init_mu);
    return rc;
}

int cpu_pool_threads(void) { return pool.count; }

static void pool_run(int n, int chunks, cpu_work work, void *arg) {
    int grain = (n + chunks * 4 - 1) / (chunks * 4);
    if (grain < 1)
        grain = 1;
    pool.work = work;
    pool.arg = arg;
    pool.n = n;
    pool.grain = grain;
    atomic_store(&pool.cursor, 0);
    atomic_store(&pool.spin, chunks >= pool.count);
    atomic_store(&pool.remaining, pool.count - 1);
    atomic_fetch_add(&pool.sequence, 1);
    for (int i = 1; i < pool.count; i++)
        if (atomic_load(&pool.slots[i].sleeping))
            wake(&pool.slots[i]);
    consume();
    while (atomic_load(&pool.remaining) != 0) {
        if (atomic_load(&pool.spin))
            spin_pause();
        else
            sched_yield();
    }
    pool.work = NULL;
}

/* InParallel (nn/parallel.go:177-191), with `limit` playing GOMAXPROCS: the
 * number of threads a call may use, so one pool times 1 and all threads. */
static void in_parallel(int n, long total_work, int limit, cpu_work work, void *arg) {
    int chunks = pool.count < limit ? pool.count : limit;
    if (chunks > n)
        chunks = n;
    if (total_work < PARALLEL_THRESHOLD)
        chunks = 1;
    if (chunks <= 1) {
        work(arg, 0, n);
        return;
    }
    pthread_mutex_lock(&pool.section);
    pool_run(n, chunks, work, arg);
    pthread_mutex_unlock(&pool.section);
}

/* ---- Q6_K (nn/dot_q6_k_amd64.s:62-125) -------------------------------- */

/* One chunk of 32 six-bit magnitudes against 32 activations: int16 pair sums,
 * then the two group scales (bytes 0..15 and 16..31) into int32 lanes. */
static inline __m256i q6_chunk(__m256i acc, __m256i mag, const int8_t *a, int16_t s_lo, int16_t s_hi) {
    const __m256i sc = _mm256_blend_epi32(_mm256_set1_epi16(s_lo), _mm256_set1_epi16(s_hi), 0xF0);
    const __m256i pairs = _mm256_maddubs_epi16(mag, _mm256_loadu_si256((const __m256i *)a));
    return _mm256_add_epi32(acc, _mm256_madd_epi16(pairs, sc));
}

static float dot_q6_k_avx2(const uint8_t *w, const int8_t *q, const int16_t *bsums, const float *kscales, int n) {
    const __m256i m4 = _mm256_set1_epi8(0x0F), m2 = _mm256_set1_epi8(0x03);
    float total = 0.0f;
    for (int b = 0; b < n / 256; b++, w += 210, q += 256, bsums += 16) {
        const __m256i sc = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(w + 192)));
        int16_t s[16];
        _mm256_storeu_si256((__m256i *)s, sc);
        __m256i acc = _mm256_setzero_si256();
        for (int h = 0; h < 2; h++) {
            const __m256i l0 = _mm256_loadu_si256((const __m256i *)(w + 64 * h));
            const __m256i l1 = _mm256_loadu_si256((const __m256i *)(w + 64 * h + 32));
            const __m256i hb = _mm256_loadu_si256((const __m256i *)(w + 128 + 32 * h));
            const int8_t *a = q + 128 * h;
            const int16_t *g = s + 8 * h;
            __m256i m;
            m = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(hb, m2), 4));
            acc = q6_chunk(acc, m, a, g[0], g[1]);
            m = _mm256_or_si256(_mm256_and_si256(l1, m4),
                                _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 2), m2), 4));
            acc = q6_chunk(acc, m, a + 32, g[2], g[3]);
            m = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                                _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 4), m2), 4));
            acc = q6_chunk(acc, m, a + 64, g[4], g[5]);
            m = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                                _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 6), m2), 4));
            acc = q6_chunk(acc, m, a + 96, g[6], g[7]);
        }
        /* recentring: 32 x sum over groups of scale x sum(q) */
        const __m256i rc = _mm256_madd_epi16(_mm256_loadu_si256((const __m256i *)bsums), sc);
        acc = _mm256_sub_epi32(acc, _mm256_slli_epi32(rc, 5));
        __m128i t = _mm_add_epi32(_mm256_extracti128_si256(acc, 1), _mm256_castsi256_si128(acc));
        t = _mm_add_epi32(t, _mm_shuffle_epi32(t, 0x4E));
        t = _mm_add_epi32(t, _mm_shuffle_epi32(t, 0xB1));
        uint16_t dh;
        memcpy(&dh, w + 208, 2);
        float f = (float)_mm_cvtsi128_si32(t);
        f = f * _cvtsh_ss(dh);
        f = f * kscales[b];
        total = total + f;
    }
    return total;
}

struct q6_args {
    const uint8_t *w;
    const int8_t *qk;
    const int16_t *bsums;
    const float *kscales;
    int cols, size, ldy;
    float *y;
};

static void q6_rows(void *p, int start, int end) {
    const struct q6_args *a = p;
    const size_t stride = (size_t)a->cols / 256 * 210;
    for (int r = start; r < end; r++)
        for (int c = 0; c < a->size; c++)
            a->y[(size_t)c * a->ldy + r] =
                dot_q6_k_avx2(a->w + r * stride, a->qk + (size_t)c * a->cols, a->bsums + (size_t)c * a->cols / 16,
                              a->kscales + (size_t)c * a->cols / 256, a->cols);
}

/* MatVecQ6_K (nn/dot_q6_k.go:64-74) on at most `threads` threads.  QK, KScales
 * and BSums in golem's layout ([column][...]); y is [size][ldy]. */
int cpu_mat_vec_q6_k(const uint8_t *w, const int8_t *qk, const int16_t *bsums, const float *kscales, int rows,
                     int cols, int size, float *y, int ldy, int threads) {
    if (cols % 256 || !pool.count)
        return -1;
    struct q6_args a = {w, qk, bsums, kscales, cols, size, ldy, y};
    in_parallel(rows, (long)rows * cols * size, threads, q6_rows, &a);
    return 0;
}

/* ---- Q4_0 (nn/dot_q4_0_amd64.s) ---------------------------------------- */

enum { BEGIN = 1, FINISH = 2 }; /* nn/dot_q4_0.go:99-104 */

/* The 32 nibbles of a block, unsigned: weights 0..15 then 16..31. */
static inline __m256i q4_unpack(const uint8_t *blk) {
    const __m128i m4 = _mm_set1_epi8(0x0F);
    const __m128i x = _mm_loadu_si128((const __m128i *)(blk + 2));
    const __m128i lo = _mm_and_si128(x, m4);
    const __m128i hi = _mm_and_si128(_mm_srli_epi16(x, 4), m4);
    return _mm256_inserti128_si256(_mm256_castsi128_si256(lo), hi, 1);
}

static inline float q4_scale(const uint8_t *blk) {
    uint16_t h;
    memcpy(&h, blk, 2);
    return _cvtsh_ss(h);
}

/* The eight int32 sums of one block against one column. */
static inline __m256 q4_column(__m256i nib, const int8_t *q) {
    const __m256i pairs = _mm256_maddubs_epi16(nib, _mm256_loadu_si256((const __m256i *)q));
    return _mm256_cvtepi32_ps(_mm256_madd_epi16(pairs, _mm256_set1_epi16(1)));
}

/* Eight lanes and a correction to one product: ((l0+l4)+(l2+l6)) +
 * ((l1+l5)+(l3+l7)) - corr (REDUCE; nn/dot_q4_0.go:108-114). */
static inline float q4_reduce(__m256 acc, float corr) {
    __m128 lo = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    const float s = _mm_cvtss_f32(lo) + _mm_cvtss_f32(_mm_shuffle_ps(lo, lo, 0x01));
    return s - corr;
}

/* dotQ4_0AVX2: state = 8 lanes + 1 correction. */
static void dot_q4_0_x1(const uint8_t *w, const int8_t *q, const float *scales, const float *corr, int n,
                        int stride, float *state, int mode) {
    __m256 acc = (mode & BEGIN) ? _mm256_setzero_ps() : _mm256_loadu_ps(state);
    float c = (mode & BEGIN) ? 0.0f : state[8];
    for (int b = 0; b < n / 32; b++) {
        const __m256i nib = q4_unpack(w);
        const float d = q4_scale(w);
        const __m256 s = _mm256_set1_ps(d * scales[0]);
        acc = _mm256_fmadd_ps(s, q4_column(nib, q), acc);
        c = c + d * corr[0];
        w += 18;
        q += (size_t)stride * 32;
        scales += stride;
        corr += stride;
    }
    if (mode & FINISH) {
        state[0] = q4_reduce(acc, c);
    } else {
        _mm256_storeu_ps(state, acc);
        state[8] = c;
    }
}

/* dotQ4_0x4AVX2 / dotQ4_0x8AVX2: `cols` consecutive columns, state = cols x 8
 * lanes then cols corrections.  The row is unpacked once per block. */
static inline void dot_q4_0_xn(const uint8_t *w, const int8_t *q, const float *scales, const float *corr, int n,
                               int stride, float *state, int mode, const int cols) {
    __m256 acc[8];
    float c[8];
    for (int j = 0; j < cols; j++) {
        acc[j] = (mode & BEGIN) ? _mm256_setzero_ps() : _mm256_loadu_ps(state + 8 * j);
        c[j] = (mode & BEGIN) ? 0.0f : state[8 * cols + j];
    }
    for (int b = 0; b < n / 32; b++) {
        const __m256i nib = q4_unpack(w);
        const float d = q4_scale(w);
        float sd[8];
        for (int j = 0; j < cols; j++) {
            sd[j] = d * scales[j];
            c[j] = c[j] + d * corr[j];  /* a multiply and an add, as x1 */
        }
        for (int j = 0; j < cols; j++)
            acc[j] = _mm256_fmadd_ps(_mm256_set1_ps(sd[j]), q4_column(nib, q + 32 * j), acc[j]);
        w += 18;
        q += (size_t)stride * 32;
        scales += stride;
        corr += stride;
    }
    for (int j = 0; j < cols; j++) {
        if (mode & FINISH) {
            state[j] = q4_reduce(acc[j], c[j]);
        } else {
            _mm256_storeu_ps(state + 8 * j, acc[j]);
            state[8 * cols + j] = c[j];
        }
    }
}

/* One column group of matVecQ4_0Rows: the kernel for `cols` columns starting
 * at column c, over the inputs starting at `block`. */
static void q4_kernel(const uint8_t *w, const int8_t *Q, const float *S, const float *C, int stride, int block,
                      int c, int n, float *state, int mode, int cols) {
    const size_t at = (size_t)block * stride + c;
    if (cols == 8)
        dot_q4_0_xn(w, Q + at * 32, S + at, C + at, n, stride, state, mode, 8);
    else if (cols == 4)
        dot_q4_0_xn(w, Q + at * 32, S + at, C + at, n, stride, state, mode, 4);
    else
        dot_q4_0_x1(w, Q + at * 32, S + at, C + at, n, stride, state, mode);
}

struct q4_args {
    const uint8_t *w;
    const int8_t *Q;
    const float *S, *C;
    int stride, size, inputs, ldy;
    float *y;
};

enum { K_TILE = 2048, ROW_TILE_BYTES = 24 * 1024, MAX_ROW_TILE = 64 }; /* nn/dot_q4_0.go:147-152 */

/* matVecQ4_0Rows (nn/dot_q4_0.go:168-270): rows [start, end). */
static void q4_rows(void *p, int start, int end) {
    const struct q4_args *a = p;
    const size_t row_bytes = (size_t)a->inputs / 32 * 18;
    const int widths[3] = {8, 4, 1};
    if (a->inputs <= K_TILE) {
        float state[72];
        int c = 0;
        for (int wi = 0; wi < 3; wi++) {
            const int cols = widths[wi];
            for (; c + cols <= a->size; c += cols)
                for (int r = start; r < end; r++) {
                    q4_kernel(a->w + r * row_bytes, a->Q, a->S, a->C, a->stride, 0, c, a->inputs, state,
                              BEGIN | FINISH, cols);
                    for (int j = 0; j < cols; j++)
                        a->y[(size_t)(c + j) * a->ldy + r] = state[j];
                }
        }
        return;
    }
    const int step_bytes = K_TILE / 32 * 18;
    int rows = ROW_TILE_BYTES / step_bytes;
    rows = rows < 1 ? 1 : rows > MAX_ROW_TILE ? MAX_ROW_TILE : rows;
    static __thread float states[MAX_ROW_TILE][72];
    for (int from = start; from < end; from += rows) {
        const int to = from + rows < end ? from + rows : end;
        int c = 0;
        for (int wi = 0; wi < 3; wi++) {
            const int cols = widths[wi];
            for (; c + cols <= a->size; c += cols) {
                for (int k = 0; k < a->inputs; k += K_TILE) {
                    const int block = k / 32, n = a->inputs - k < K_TILE ? a->inputs - k : K_TILE;
                    const int mode = (k == 0 ? BEGIN : 0) | (k + n >= a->inputs ? FINISH : 0);
                    for (int r = from; r < to; r++)
                        q4_kernel(a->w + r * row_bytes + (size_t)block * 18, a->Q, a->S, a->C, a->stride, block, c,
                                  n, states[r - from], mode, cols);
                }
                for (int r = from; r < to; r++)
                    for (int j = 0; j < cols; j++)
                        a->y[(size_t)(c + j) * a->ldy + r] = states[r - from][j];
            }
        }
    }
}

/* MatVecQ4_0 (nn/dot_q4_0.go:117-124) on at most `threads` threads.  Q,
 * Scales and Corr in golem's interleaved layout with stride = size; y is
 * [size][ldy]. */
int cpu_mat_vec_q4_0(const uint8_t *w, const int8_t *Q, const float *S, const float *C, int rows, int inputs,
                     int size, float *y, int ldy, int threads) {
    if (inputs % 32 || !pool.count)
        return -1;
    struct q4_args a = {w, Q, S, C, size, size, inputs, ldy, y};
    in_parallel(rows, (long)rows * inputs * size, threads, q4_rows, &a);
    return 0;
}

/* ---- the packed product (nn/pack_q4_0.go, nn/pack_q4_0_amd64.s) ----------
 *
 * Eight rows interleaved per group of blocks (144 bytes a block: the rows'
 * eight fp16 scales, then four 32-byte chunks of eight inputs; byte s*8+j of
 * chunk g holds row {0,1,4,5}[s] in its low nibble and row {2,3,6,7}[s] in
 * its high one, at input 8g+j).  dotPackedQ4_0x4AVX2 (:99-160) multiplies a
 * group against four columns: per block the nibbles are split into eight
 * registers once; per column the eight activation bytes of a chunk are
 * broadcast to its four slots, VPMADDUBSW'd against the low and the high
 * nibbles, the int16 pairs summed over the four chunks, widened by VPMADDWD
 * against ones and folded by one VPHADDD into the eight rows in order; then
 * acc += float(sums) * (act_scale * row_scale) and acc -= corr * row_scale,
 * both fused.  dotPackedQ4_0AVX2 is the same for one column. */
static inline void packed_unpack(const uint8_t *blk, __m256i nib[8], __m256 *rs) {
    *rs = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)blk));
    const __m256i mask = _mm256_set1_epi8(0x0F);
    for (int g = 0; g < 4; g++) {
        const __m256i c = _mm256_loadu_si256((const __m256i *)(blk + 16 + 32 * g));
        nib[2 * g] = _mm256_and_si256(c, mask);
        nib[2 * g + 1] = _mm256_and_si256(_mm256_srli_epi16(c, 4), mask);
    }
}

static inline __m256 packed_sums(const __m256i nib[8], const int8_t *q) {
    __m256i lo = _mm256_setzero_si256(), hi = _mm256_setzero_si256();
    for (int g = 0; g < 4; g++) {
        const __m256i a = _mm256_set1_epi64x(*(const long long *)(q + 8 * g));
        const __m256i l = _mm256_maddubs_epi16(nib[2 * g], a), h = _mm256_maddubs_epi16(nib[2 * g + 1], a);
        lo = g == 0 ? l : _mm256_add_epi16(lo, l);
        hi = g == 0 ? h : _mm256_add_epi16(hi, h);
    }
    const __m256i ones = _mm256_set1_epi16(1);
    return _mm256_cvtepi32_ps(_mm256_hadd_epi32(_mm256_madd_epi16(lo, ones), _mm256_madd_epi16(hi, ones)));
}

/* One group of eight rows against `cols` (4 or 1) columns from column c,
 * over n inputs from `block`; state: cols x 8 running sums. */
static void packed_kernel(const uint8_t *w, const int8_t *Q, const float *S, const float *C, int stride, int block,
                          int c, int n, float *state, int mode, int cols) {
    __m256 acc[4];
    for (int j = 0; j < cols; j++)
        acc[j] = (mode & BEGIN) ? _mm256_setzero_ps() : _mm256_loadu_ps(state + 8 * j);
    for (int b = 0; b < n / 32; b++) {
        __m256i nib[8];
        __m256 rs;
        packed_unpack(w + (size_t)b * 144, nib, &rs);
        const size_t at = (size_t)(block + b) * stride + c;
        for (int j = 0; j < cols; j++) {
            const __m256 sums = packed_sums(nib, Q + (at + j) * 32);
            const __m256 sc = _mm256_mul_ps(_mm256_set1_ps(S[at + j]), rs);
            acc[j] = _mm256_fmadd_ps(sums, sc, acc[j]);
            acc[j] = _mm256_fnmadd_ps(_mm256_set1_ps(C[at + j]), rs, acc[j]);
        }
    }
    for (int j = 0; j < cols; j++)
        _mm256_storeu_ps(state + 8 * j, acc[j]);
}

struct packed_args {
    const uint8_t *w;
    const int8_t *Q;
    const float *S, *C;
    int size, inputs, ldy;
    float *y;
};

enum { MAX_GROUP_TILE = 8 }; /* nn/pack_q4_0.go:147-152 */

/* matVecPackedQ4_0Rows (nn/pack_q4_0.go:153-221): rows [start, end), a
 * group computed whole and written in part. */
static void packed_rows(void *p, int start, int end) {
    const struct packed_args *a = p;
    const size_t group_bytes = (size_t)a->inputs / 32 * 144;
    const int first = start / 8, last = (end + 7) / 8;
    const int steps = K_TILE < a->inputs ? K_TILE : a->inputs;
    const int step_bytes = steps / 32 * 144;
    int tile = ROW_TILE_BYTES / step_bytes;
    tile = tile < 1 ? 1 : tile > MAX_GROUP_TILE ? MAX_GROUP_TILE : tile;
    float four[MAX_GROUP_TILE][32], one[MAX_GROUP_TILE][8];
    for (int from = first; from < last; from += tile) {
        const int to = from + tile < last ? from + tile : last;
        int c = 0;
        for (int wi = 0; wi < 2; wi++) {
            const int cols = wi == 0 ? 4 : 1;
            for (; c + cols <= a->size; c += cols) {
                for (int k = 0; k < a->inputs; k += steps) {
                    const int block = k / 32, n = a->inputs - k < steps ? a->inputs - k : steps;
                    const int mode = (k == 0 ? BEGIN : 0) | (k + n >= a->inputs ? FINISH : 0);
                    for (int g = from; g < to; g++)
                        packed_kernel(a->w + (size_t)g * group_bytes + (size_t)block * 144, a->Q, a->S, a->C,
                                      a->size, block, c, n, cols == 4 ? four[g - from] : one[g - from], mode, cols);
                }
                for (int g = from; g < to; g++)
                    for (int j = 0; j < cols; j++)
                        for (int r = 0; r < 8; r++) {
                            const int row = 8 * g + r;
                            if (row >= start && row < end)
                                a->y[(size_t)(c + j) * a->ldy + row] =
                                    (cols == 4 ? four[g - from] : one[g - from])[8 * j + r];
                        }
            }
        }
    }
}

/* The packed product of golem's loader (whole groups of eight rows) over a
 * batch in golem's interleaved layout, on at most `threads` threads. */
int cpu_mat_vec_packed_q4_0(const uint8_t *packed, const int8_t *Q, const float *S, const float *C, int rows,
                            int inputs, int size, float *y, int ldy, int threads) {
    if (inputs % 32 || rows % 8 || !pool.count)
        return -1;
    struct packed_args a = {packed, Q, S, C, size, inputs, ldy, y};
    in_parallel(rows, (long)rows * inputs * size, threads, packed_rows, &a);
    return 0;
}

/* The single kernels, for the tests: one row against columns [c, c+cols). */
void cpu_dot_q4_0(const uint8_t *w, const int8_t *Q, const float *S, const float *C, int stride, int block, int c,
                  int n, float *state, int mode, int cols) {
    q4_kernel(w, Q, S, C, stride, block, c, n, state, mode, cols);
}

float cpu_dot_q6_k(const uint8_t *w, const int8_t *q, const int16_t *bsums, const float *kscales, int n) {
    return dot_q6_k_avx2(w, q, bsums, kscales, n);
}

/* ---- gemma's MoE feed-forward (gemma/moe.go:34-180) ------------------------
 *
 * Route and ExpertFFN as golem runs them on x86, for config 4's CPU figure:
 *   Route          per position RMSNormPlain (nn/ops.go:195-214, the float64
 *                  sum left to right) times 1/sqrt(Dim) (RouterScale ones),
 *                  then the F32 router through Matrix.rows' F32 case --
 *                  dotF32AVX2 (nn/dot_f32_amd64.s:43-113: four accumulators
 *                  of eight lanes, the eights, the remainder, nothing fused)
 *                  in a section over the router's rows -- then
 *                  chooseExperts (gemma/moe.go:62-88);
 *   ExpertFFN      a section over positions quantising each input
 *                  (Batch.quantizeBlock, nn/batch.go:109-143), a section over
 *                  the (position, slot) units -- the expert's gate|up rows
 *                  through matVecQ4_0Rows (the row layout: expert stacks are
 *                  not repacked), GELUTable(gate) * up, its Q8_0, the down
 *                  rows -- and a section over positions summing the units
 *                  with Axpy (the FMA form, nn/kernel_amd64.s:134-197),
 *                  DownScale ones. */

/* dotF32AVX2 */
static float dot_f32_avx2(const float *a, const float *b, int n) {
    __m256 y0 = _mm256_setzero_ps(), y1 = _mm256_setzero_ps(), y2 = _mm256_setzero_ps(), y3 = _mm256_setzero_ps();
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        y0 = _mm256_add_ps(y0, _mm256_mul_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i)));
        y1 = _mm256_add_ps(y1, _mm256_mul_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8)));
        y2 = _mm256_add_ps(y2, _mm256_mul_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16)));
        y3 = _mm256_add_ps(y3, _mm256_mul_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24)));
    }
    y0 = _mm256_add_ps(y0, y1);
    y2 = _mm256_add_ps(y2, y3);
    y0 = _mm256_add_ps(y0, y2);
    for (; i + 8 <= n; i += 8)
        y0 = _mm256_add_ps(y0, _mm256_mul_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i)));
    __m128 x = _mm_add_ps(_mm256_castps256_ps128(y0), _mm256_extractf128_ps(y0, 1));
    x = _mm_add_ps(x, _mm_movehl_ps(x, x));
    x = _mm_add_ss(x, _mm_shuffle_ps(x, x, 0x01));
    float s = _mm_cvtss_f32(x);
    for (; i < n; i++)
        s += a[i] * b[i];
    return s;
}

/* Batch.quantizeBlock for one column's n inputs (golem's generic Go: the
 * only form it has). */
static inline int32_t nearest(float f) {
    float s = f + 12582912.0f;
    int32_t u;
    memcpy(&u, &s, 4);
    return (u & 0x007fffff) - 0x00400000;
}
static void quantize_column(const float *x, int n, int8_t *q, float *scales, float *corr) {
    for (int b = 0; b < n / 32; b++) {
        const float *v = x + 32 * b;
        float peak = 0;
        for (int i = 0; i < 32; i++) {
            const float a = v[i] < 0 ? -v[i] : v[i];
            if (a > peak)
                peak = a;
        }
        if (peak == 0) {
            scales[b] = corr[b] = 0;
            memset(q + 32 * b, 0, 32);
            continue;
        }
        const float scale = peak / 127, inverse = 127 / peak;
        scales[b] = _cvtsh_ss(_cvtss_sh(scale, _MM_FROUND_TO_NEAREST_INT));
        int32_t sum = 0;
        for (int i = 0; i < 32; i++) {
            int32_t k = nearest(v[i] * inverse);
            k = k > 127 ? 127 : k < -128 ? -128 : k;
            q[32 * b + i] = (int8_t)k;
            sum += k;
        }
        corr[b] = 8 * scales[b] * (float)sum;
    }
}

struct moe_cpu {
    const float *router;              /* [E][D] */
    const uint8_t *gate_up, *down;    /* row-layout Q4_0 stacks */
    const float *gelu;                /* golem's 65536-entry table, indexed by the fp16 bits */
    int D, F, E, k, batch;
    const float *resid;               /* [batch][D]: the router's and the experts' input */
    float *rin;                       /* [batch][D] scratch */
    float *logits;                    /* [batch][E] */
    int32_t *ids;                     /* [batch][k] */
    float *weights;                   /* [batch][k] */
    int8_t *xq;                       /* [batch][D], scales / corr [batch][D/32] */
    float *xs, *xc;
    float *gu;                        /* [units][2F] */
    int8_t *mq;                       /* [units][F], scales / corr [units][F/32] */
    float *ms, *mc;
    float *partial;                   /* [units][D] */
    float *out;                       /* [batch][D] */
};

static void moe_norm_section(void *p, int start, int end) {
    struct moe_cpu *m = p;
    const float scale = (float)(1 / __builtin_sqrt((double)m->D));
    for (int t = start; t < end; t++) {
        float *x = m->rin + (size_t)t * m->D;
        memcpy(x, m->resid + (size_t)t * m->D, sizeof(float) * m->D);
        double s = 0;
        for (int i = 0; i < m->D; i++)
            s += (double)(x[i] * x[i]);
        const float mean = (float)(s / (double)m->D);
        const float r = (float)(1 / __builtin_sqrt((double)(mean + 1e-6f)));
        for (int i = 0; i < m->D; i++)
            x[i] = (x[i] * r) * (scale * 1.0f);
        /* the router's input is quantised too (its F32 product reads the floats) */
        quantize_column(x, m->D, m->xq + (size_t)t * m->D, m->xs + (size_t)t * m->D / 32,
                        m->xc + (size_t)t * m->D / 32);
    }
}

static void moe_router_section(void *p, int start, int end) {
    struct moe_cpu *m = p;
    for (int t = 0; t < m->batch; t++)
        for (int e = start; e < end; e++)
            m->logits[(size_t)t * m->E + e] =
                dot_f32_avx2(m->router + (size_t)e * m->D, m->rin + (size_t)t * m->D, m->D);
}

static void moe_choose(struct moe_cpu *m) {
    for (int t = 0; t < m->batch; t++) {
        const float *l = m->logits + (size_t)t * m->E;
        int32_t *ids = m->ids + (size_t)t * m->k;
        float *w = m->weights + (size_t)t * m->k;
        for (int k = 0; k < m->k; k++) {
            int best = -1;
            for (int e = 0; e < m->E; e++) {
                int taken = 0;
                for (int j = 0; j < k; j++)
                    taken |= ids[j] == e;
                if (!taken && (best < 0 || l[e] > l[best]))
                    best = e;
            }
            ids[k] = best;
        }
        const float top = l[ids[0]];
        float total = 0;
        for (int k = 0; k < m->k; k++) {
            w[k] = (float)__builtin_exp((double)(l[ids[k]] - top));
            total += w[k];
        }
        for (int k = 0; k < m->k; k++)
            w[k] /= total;
    }
}

static void moe_quantize_section(void *p, int start, int end) {
    struct moe_cpu *m = p;
    for (int t = start; t < end; t++)
        quantize_column(m->resid + (size_t)t * m->D, m->D, m->xq + (size_t)t * m->D, m->xs + (size_t)t * m->D / 32,
                        m->xc + (size_t)t * m->D / 32);
}

static inline float gelu_lookup(const float *table, float x) {
    if (x <= -10.0f)
        return 0.0f;
    if (x >= 10.0f)
        return x;
    return table[_cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT)];
}

static void moe_units_section(void *p, int start, int end) {
    struct moe_cpu *m = p;
    const int D = m->D, F = m->F;
    const size_t gu_bytes = (size_t)2 * F * (D / 32) * 18, dn_bytes = (size_t)D * (F / 32) * 18;
    for (int u = start; u < end; u++) {
        const int t = u / m->k, id = m->ids[u];
        float *gu = m->gu + (size_t)u * 2 * F;
        struct q4_args a = {m->gate_up + (size_t)id * gu_bytes, m->xq + (size_t)t * D, m->xs + (size_t)t * D / 32,
                            m->xc + (size_t)t * D / 32, 1, 1, D, 2 * F, gu};
        q4_rows(&a, 0, 2 * F);
        float *mid = gu;  /* gate, then gate * up in place */
        for (int i = 0; i < F; i++)
            mid[i] = gelu_lookup(m->gelu, gu[i]) * gu[F + i];
        int8_t *mq = m->mq + (size_t)u * F;
        float *ms = m->ms + (size_t)u * F / 32, *mc = m->mc + (size_t)u * F / 32;
        quantize_column(mid, F, mq, ms, mc);
        struct q4_args b = {m->down + (size_t)id * dn_bytes, mq, ms, mc, 1, 1, F, D, m->partial + (size_t)u * D};
        q4_rows(&b, 0, D);
    }
}

static void moe_reduce_section(void *p, int start, int end) {
    struct moe_cpu *m = p;
    for (int t = start; t < end; t++) {
        float *o = m->out + (size_t)t * m->D;
        memset(o, 0, sizeof(float) * m->D);
        for (int k = 0; k < m->k; k++) {
            const __m256 w = _mm256_set1_ps(m->weights[(size_t)t * m->k + k] * 1.0f);
            const float *src = m->partial + ((size_t)t * m->k + k) * m->D;
            int i = 0;
            for (; i + 8 <= m->D; i += 8)
                _mm256_storeu_ps(o + i, _mm256_fmadd_ps(w, _mm256_loadu_ps(src + i), _mm256_loadu_ps(o + i)));
            for (; i < m->D; i++)
                o[i] += m->weights[(size_t)t * m->k + k] * src[i];
        }
    }
}

/* Route + ExpertFFN for `batch` positions on at most `threads` threads;
 * scratch is caller-owned (sizes as the struct says). */
int cpu_moe_ffn(const float *router, const uint8_t *gate_up, const uint8_t *down, const float *gelu, int D, int F,
                int E, int k, int batch, const float *resid, float *rin, float *logits, int32_t *ids, float *weights,
                int8_t *xq, float *xs, float *xc, float *gu, int8_t *mq, float *ms, float *mc, float *partial,
                float *out, int threads) {
    if (!pool.count || D % 32 || F % 32)
        return -1;
    struct moe_cpu m = {router, gate_up, down, gelu, D, F, E, k, batch, resid, rin, logits, ids, weights,
                        xq, xs, xc, gu, mq, ms, mc, partial, out};
    enum { PER_POSITION = 24 }; /* gemma/block.go:104 */
    in_parallel(batch, (long)batch * D * PER_POSITION, threads, moe_norm_section, &m);
    in_parallel(E, (long)batch * E * D, threads, moe_router_section, &m);
    moe_choose(&m);
    in_parallel(batch, (long)batch * D * PER_POSITION, threads, moe_quantize_section, &m);
    const int units = batch * k;
    in_parallel(units, (long)units * F * D * 2, threads, moe_units_section, &m);
    in_parallel(batch, (long)batch * k * D, threads, moe_reduce_section, &m);
    return 0;
}

/* ---- qwen's decode token (qwen/block.go:32-102, qwen/attention.go:34-127) --
 *
 * One position through every block and the tied Q6_K head, as golem runs it
 * on x86: the pre-norms (RMSNormPlain with the block's gain, then the Q8_0
 * form), the head section (a unit a query head or a key-value head: its 128
 * rows of the packed products through matVecPackedQ4_0Rows, the head norm,
 * RoPE, fp16 rounding, the cache store), the attention section (a unit a
 * query head: DotF32 scores through dotF32AVX2, SoftmaxInPlace in float64
 * exp, fp16 probabilities, Axpy of the cached values, the head's Q8_0), O,
 * the FFN section (a unit a 32-row stretch of Gate and of Up, SwiGLU with
 * ggml's expf (nn/swiglu.go:31-82) and the stretch's Q8_0), Down, the
 * residual adds; then the final norm, QuantizeK and MatVecQ6_K. */

static void rms_norm(float *x, const float *gain, int n, float eps) {
    double s = 0;
    for (int i = 0; i < n; i++)
        s += (double)(x[i] * x[i]);
    const float mean = (float)(s / (double)n);
    const float r = (float)(1 / __builtin_sqrt((double)(mean + eps)));
    for (int i = 0; i < n; i++)
        x[i] = gain ? (x[i] * r) * gain[i] : x[i] * r;
}

static inline float round_half(float v) { return _cvtsh_ss(_cvtss_sh(v, _MM_FROUND_TO_NEAREST_INT)); }

/* ggml's expf as golem restates it (nn/swiglu.go:31-74) */
static float ggml_expf(float x) {
    const float shift = 0x1.8p23f, log2e = 0x1.715476p+0f, ln2hi = 0x1.62e4p-1f, ln2lo = 0x1.7f7d1cp-20f;
    const float c0 = 0x1.ffffecp-1f, c1 = 0x1.fffdb6p-2f, c2 = 0x1.555e66p-3f, c3 = 0x1.573e2ep-5f,
                c4 = 0x1.0e4020p-7f;
    const float z = x * log2e + shift, n = z - shift;
    if (n > 126 || n < -126)
        return (float)__builtin_exp((double)x);
    const float b = x - n * ln2hi - n * ln2lo;
    uint32_t zu, one;
    const float onef = 1.0f;
    memcpy(&zu, &z, 4);
    memcpy(&one, &onef, 4);
    const uint32_t ku = (zu << 23) + one;
    float k;
    memcpy(&k, &ku, 4);
    const float u = b * b;
    const float j = ((c4 * b + c3) * u + (c2 * b + c1)) * u + c0 * b;
    return j * k + k;
}

/* Batch.QuantizeK (nn/batch.go:159-213) of one column */
static void quantize_k(const float *x, int n, int8_t *q, float *kscales, int16_t *bsums) {
    for (int b = 0; b < n / 256; b++) {
        const float *v = x + 256 * b;
        float peak = 0, extreme = 0;
        for (int i = 0; i < 256; i++) {
            const float a = v[i] < 0 ? -v[i] : v[i];
            if (a > peak) {
                peak = a;
                extreme = v[i];
            }
        }
        if (peak == 0) {
            kscales[b] = 0;
            memset(q + 256 * b, 0, 256);
            for (int g = 0; g < 16; g++)
                bsums[16 * b + g] = 0;
            continue;
        }
        const float inverse = -128 / extreme;
        for (int g = 0; g < 16; g++) {
            int32_t s = 0;
            for (int i = 16 * g; i < 16 * g + 16; i++) {
                int32_t k = nearest(v[i] * inverse);
                k = k > 127 ? 127 : k;
                q[256 * b + i] = (int8_t)k;
                s += k;
            }
            bsums[16 * b + g] = (int16_t)s;
        }
        kscales[b] = 1 / inverse;
    }
}

enum { QL_Q, QL_K, QL_V, QL_O, QL_GATE, QL_UP, QL_DOWN, QL_ATTN_NORM, QL_FFN_NORM, QL_Q_NORM, QL_K_NORM, QL_KC, QL_VC,
       QL_COUNT };

struct qwen_cpu {
    void *const *layer;  /* [layers][QL_COUNT] */
    int D, F, H, KV, HD, ctx, pos;
    float eps, scale;
    const float *cos, *sin;  /* the rotation at pos, [HD/2] */
    int8_t *nq; float *ns, *nc;          /* the normed input's Q8_0 [D] */
    float *qh;                           /* [H][HD] rounded queries */
    float *hk, *hv;                      /* [KV][HD] scratch for the projections */
    int8_t *sq; float *ss, *sc;          /* the heads' Q8_0 [H * HD] */
    float *set;                          /* [H * HD] */
    float *scores;                       /* [H][ctx] */
    float *gate, *up;                    /* [F] */
    int8_t *mq; float *msc, *mc;         /* mid's Q8_0 [F] */
    int L;
};

static void packed_range(const uint8_t *w, const int8_t *Q, const float *S, const float *C, int inputs, float *y,
                         int start, int end) {
    struct packed_args a = {w, Q, S, C, 1, inputs, 0, y};
    packed_rows(&a, start, end);
}

static void qwen_heads_section(void *p, int start, int end) {
    struct qwen_cpu *m = p;
    void *const *lw = m->layer + (size_t)m->L * QL_COUNT;
    const int HD = m->HD, half = HD / 2;
    for (int u = start; u < end; u++) {
        const int is_q = u < m->H, h = is_q ? u : u - m->H;
        float *head = is_q ? m->qh + (size_t)h * HD : m->hk + (size_t)h * HD;
        /* the head's rows; golem's scratch rows are indexed by the matrix row */
        packed_range(lw[is_q ? QL_Q : QL_K], m->nq, m->ns, m->nc, m->D, head - (size_t)h * HD, h * HD, (h + 1) * HD);
        rms_norm(head, lw[is_q ? QL_Q_NORM : QL_K_NORM], HD, m->eps);
        for (int i = 0; i < half; i++) {
            const float re = head[i], im = head[i + half];
            head[i] = re * m->cos[i] - im * m->sin[i];
            head[i + half] = re * m->sin[i] + im * m->cos[i];
        }
        for (int i = 0; i < HD; i++)
            head[i] = round_half(head[i]);
        if (!is_q) {
            float *vh = m->hv + (size_t)h * HD;
            packed_range(lw[QL_V], m->nq, m->ns, m->nc, m->D, vh - (size_t)h * HD, h * HD, (h + 1) * HD);
            float *kc = (float *)lw[QL_KC] + ((size_t)m->pos * m->KV + h) * HD;
            float *vc = (float *)lw[QL_VC] + ((size_t)m->pos * m->KV + h) * HD;
            for (int i = 0; i < HD; i++) {
                kc[i] = head[i];
                vc[i] = round_half(vh[i]);
            }
        }
    }
}

static void qwen_attend_section(void *p, int start, int end) {
    struct qwen_cpu *m = p;
    void *const *lw = m->layer + (size_t)m->L * QL_COUNT;
    const int HD = m->HD, n = m->pos + 1;
    const float *kc = lw[QL_KC], *vc = lw[QL_VC];
    for (int h = start; h < end; h++) {
        const int kv = h / (m->H / m->KV);
        float *s = m->scores + (size_t)h * m->ctx;
        const float *q = m->qh + (size_t)h * HD;
        float mx = -__builtin_inff();
        for (int p2 = 0; p2 < n; p2++) {
            s[p2] = m->scale * dot_f32_avx2(q, kc + ((size_t)p2 * m->KV + kv) * HD, HD);
            if (s[p2] > mx)
                mx = s[p2];
        }
        float total = 0;
        for (int p2 = 0; p2 < n; p2++) {
            s[p2] = (float)__builtin_exp((double)(s[p2] - mx));
            total += s[p2];
        }
        for (int p2 = 0; p2 < n; p2++)
            s[p2] = round_half(s[p2] / total);
        float *dst = m->set + (size_t)h * HD;
        memset(dst, 0, sizeof(float) * HD);
        for (int p2 = 0; p2 < n; p2++) {
            const __m256 a = _mm256_set1_ps(s[p2]);
            const float *src = vc + ((size_t)p2 * m->KV + kv) * HD;
            for (int i = 0; i < HD; i += 8)
                _mm256_storeu_ps(dst + i, _mm256_fmadd_ps(a, _mm256_loadu_ps(src + i), _mm256_loadu_ps(dst + i)));
        }
        quantize_column(dst, HD, m->sq + (size_t)h * HD, m->ss + (size_t)h * HD / 32, m->sc + (size_t)h * HD / 32);
    }
}

static void qwen_ffn_section(void *p, int start, int end) {
    struct qwen_cpu *m = p;
    void *const *lw = m->layer + (size_t)m->L * QL_COUNT;
    const int from = 32 * start, to = 32 * end;
    packed_range(lw[QL_GATE], m->nq, m->ns, m->nc, m->D, m->gate, from, to);
    packed_range(lw[QL_UP], m->nq, m->ns, m->nc, m->D, m->up, from, to);
    for (int i = from; i < to; i++) {
        const float g = m->gate[i];
        m->gate[i] = g / (1 + ggml_expf(-g)) * m->up[i];
    }
    quantize_column(m->gate + from, to - from, m->mq + from, m->msc + from / 32, m->mc + from / 32);
}

static void qwen_rows_o(void *p, int start, int end) {
    struct qwen_cpu *m = p;
    void *const *lw = m->layer + (size_t)m->L * QL_COUNT;
    packed_range(lw[QL_O], m->sq, m->ss, m->sc, m->H * m->HD, m->gate /* attn out, D <= F */, start, end);
}

static void qwen_rows_down(void *p, int start, int end) {
    struct qwen_cpu *m = p;
    void *const *lw = m->layer + (size_t)m->L * QL_COUNT;
    packed_range(lw[QL_DOWN], m->mq, m->msc, m->mc, m->F, m->up /* ffn out, D <= F */, start, end);
}

/* One decode token: x [D] is the embedding row in and the hidden state after
 * the final norm out; logits [vocab] through the Q6_K head. */
int cpu_qwen_token(void *const *layers, int nlayers, int D, int F, int H, int KV, int HD, int ctx, int pos, float eps,
                   const float *cos, const float *sin, const float *output_norm, const uint8_t *head, int vocab,
                   float *x, float *logits, int threads) {
    if (!pool.count || pos >= ctx || D > F || H * HD > F)
        return -1;
    enum { PER_POSITION = 24 }; /* qwen/block.go:30 */
    const int QD = H * HD;
    struct qwen_cpu m = {0};
    m.layer = layers;
    m.D = D, m.F = F, m.H = H, m.KV = KV, m.HD = HD, m.ctx = ctx, m.pos = pos;
    m.eps = eps;
    m.scale = (float)(1 / __builtin_sqrt((double)HD));
    m.cos = cos, m.sin = sin;
    float *normed = malloc(sizeof(float) * D);
    m.nq = malloc(D), m.ns = malloc(sizeof(float) * D / 32), m.nc = malloc(sizeof(float) * D / 32);
    m.qh = malloc(sizeof(float) * QD), m.hk = malloc(sizeof(float) * KV * HD), m.hv = malloc(sizeof(float) * KV * HD);
    m.sq = malloc(QD), m.ss = malloc(sizeof(float) * QD / 32), m.sc = malloc(sizeof(float) * QD / 32);
    m.set = malloc(sizeof(float) * QD), m.scores = malloc(sizeof(float) * H * ctx);
    m.gate = malloc(sizeof(float) * F), m.up = malloc(sizeof(float) * F);
    m.mq = malloc(F), m.msc = malloc(sizeof(float) * F / 32), m.mc = malloc(sizeof(float) * F / 32);
    for (int L = 0; L < nlayers; L++) {
        void *const *lw = layers + (size_t)L * QL_COUNT;
        m.L = L;
        memcpy(normed, x, sizeof(float) * D);
        rms_norm(normed, lw[QL_ATTN_NORM], D, eps);
        quantize_column(normed, D, m.nq, m.ns, m.nc);
        in_parallel(H + KV, (long)(H + KV) * HD * D, threads, qwen_heads_section, &m);
        in_parallel(H, 2L * H * (pos + 1) * HD, threads, qwen_attend_section, &m);
        in_parallel(D, (long)D * QD, threads, qwen_rows_o, &m);  /* O.MatVecBatch */
        for (int i = 0; i < D; i++)
            x[i] += m.gate[i];
        memcpy(normed, x, sizeof(float) * D);
        rms_norm(normed, lw[QL_FFN_NORM], D, eps);
        quantize_column(normed, D, m.nq, m.ns, m.nc);
        in_parallel(F / 32, 2L * F * D, threads, qwen_ffn_section, &m);
        in_parallel(D, (long)D * F, threads, qwen_rows_down, &m);  /* Down.MatVecBatch */
        for (int i = 0; i < D; i++)
            x[i] += m.up[i];
        (void)PER_POSITION;  /* a batch of one: the per-position sections run on the caller */
    }
    rms_norm(x, output_norm, D, eps);
    int8_t *kq = malloc(D);
    float *ks = malloc(sizeof(float) * D / 256);
    int16_t *bs = malloc(sizeof(int16_t) * D / 16);
    quantize_k(x, D, kq, ks, bs);
    struct q6_args a = {head, kq, bs, ks, D, 1, vocab, logits};
    in_parallel(vocab, (long)vocab * D, threads, q6_rows, &a);
    free(kq), free(ks), free(bs), free(normed);
    free(m.nq), free(m.ns), free(m.nc), free(m.qh), free(m.hk), free(m.hv), free(m.sq), free(m.ss), free(m.sc);
    free(m.set), free(m.scores), free(m.gate), free(m.up), free(m.mq), free(m.msc), free(m.mc);
    return 0;
}

/* dotF32AVX2, for the tests */
float cpu_dot_f32(const float *a, const float *b, int n) { return n == 0 ? 0.0f : dot_f32_avx2(a, b, n); }
