/*
 * px_datagen.c -- deterministic synthetic workloads for tests and benchmarks.
 *
 * Host-only; built as proxima_amd/libpx_datagen.so. No counterpart in the reference's
 * FFI: the reference regenerates its inputs from SplitMix64 seeds in each test
 * (crates/core/src/flat.rs:238-250, crates/core/src/pq.rs:404-407,
 * crates/core/examples/gpu_knn.rs:349-361) and uses numpy default_rng in Python.
 *
 * Counter form of SplitMix64: stream element i of seed s is
 *   mix(s + (i + 1) * 0x9E3779B97F4A7C15),
 * which is exactly the i-th output of the reference's sequential SplitMix
 * (pq.rs:27-33), so any element can be produced independently and in parallel.
 * No libm call sits in any sampling path: every generator is bit-reproducible.
 */
#include <math.h>
#include <stdint.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define PX_GOLDEN 0x9E3779B97F4A7C15ull

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* i-th output (0-based) of SplitMix64 seeded with seed */
static inline uint64_t stream_at(uint64_t seed, uint64_t i) {
    return mix64(seed + (i + 1) * PX_GOLDEN);
}

uint64_t px_gen_stream_at(uint64_t seed, uint64_t i) { return stream_at(seed, i); }

/* The reference's test generator, (z as f32 / u64::MAX as f32) * 2.0 - 1.0
 * (flat.rs:242-247, gpu_knn.rs:349-361): uniform in [-1, 1]. */
void px_gen_uniform_pm1(uint64_t seed, int64_t start, int64_t count, float* out) {
    const float denom = (float)UINT64_MAX;
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < count; ++e) {
        uint64_t z = stream_at(seed, (uint64_t)(start + e));
        float u = (float)z / denom;
        out[e] = u * 2.0f - 1.0f;
    }
}

/* Irwin-Hall(12) approximation of N(0,1): element e sums the twelve 24-bit uniforms
 * at stream positions 12e .. 12e+11 as integers, then (sum * 2^-24 - 6) in double,
 * rounded once to f32. Integer arithmetic up to the last step: host-independent. */
void px_gen_gaussian(uint64_t seed, int64_t start, int64_t count, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < count; ++e) {
        uint64_t base = (uint64_t)(start + e) * 12u;
        uint64_t s = 0;
        for (uint64_t t = 0; t < 12; ++t) s += stream_at(seed, base + t) >> 40;
        double g = (double)s * (1.0 / 16777216.0) - 6.0;
        out[e] = (float)g;
    }
}

/* floor(2^32 * (1 - exp(-(x+1)/20))) for x = 0..254 and 2^32 for x = 255: the CDF of
 * floor(Exp(mean 20)) clipped to [0, 255], as 32-bit thresholds (P(0) ~ 4.9%,
 * mean ~ 19.5). Committed as constants so that sampling never calls libm. */
static const uint64_t k_sift_thresholds[256] = {
    209468026ull, 408720177ull, 598254685ull, 778545487ull, 950043402ull,
    1113177265ull, 1268354996ull, 1415964620ull, 1556375237ull, 1689937948ull,
    1816986728ull, 1937839267ull, 2052797757ull, 2162149656ull, 2266168400ull,
    2365114089ull, 2459234141ull, 2548763903ull, 2633927248ull, 2714937127ull,
    2791996107ull, 2865296877ull, 2935022726ull, 3001348006ull, 3064438563ull,
    3124452157ull, 3181538854ull, 3235841400ull, 3287495580ull, 3336630555ull,
    3383369189ull, 3427828354ull, 3470119219ull, 3510347534ull, 3548613891ull,
    3585013977ull, 3619638808ull, 3652574967ull, 3683904811ull, 3713706680ull,
    3742055095ull, 3769020941ull, 3794671647ull, 3819071354ull, 3842281073ull,
    3864358841ull, 3885359863ull, 3905336653ull, 3924339164ull, 3942414911ull,
    3959609094ull, 3975964706ull, 3991522646ull, 4006321816ull, 4020399222ull,
    4033790065ull, 4046527829ull, 4058644365ull, 4070169970ull, 4081133465ull,
    4091562264ull, 4101482445ull, 4110918812ull, 4119894963ull, 4128433341ull,
    4136555298ull, 4144281142ull, 4151630192ull, 4158620825ull, 4165270521ull,
    4171595908ull, 4177612801ull, 4183336247ull, 4188780558ull, 4193959346ull,
    4198885562ull, 4203571523ull, 4208028948ull, 4212268981ull, 4216302225ull,
    4220138766ull, 4223788197ull, 4227259642ull, 4230561783ull, 4233702877ull,
    4236690778ull, 4239532958ull, 4242236522ull, 4244808232ull, 4247254519ull,
    4249581498ull, 4251794990ull, 4253900528ull, 4255903378ull, 4257808548ull,
    4259620801ull, 4261344670ull, 4262984465ull, 4264544286ull, 4266028033ull,
    4267439418ull, 4268781968ull, 4270059042ull, 4271273832ull, 4272429376ull,
    4273528563ull, 4274574142ull, 4275568728ull, 4276514807ull, 4277414746ull,
    4278270794ull, 4279085092ull, 4279859676ull, 4280596483ull, 4281297356ull,
    4281964047ull, 4282598223ull, 4283201470ull, 4283775296ull, 4284321136ull,
    4284840355ull, 4285334252ull, 4285804061ull, 4286250957ull, 4286676058ull,
    4287080427ull, 4287465074ull, 4287830961ull, 4288179004ull, 4288510073ull,
    4288824996ull, 4289124559ull, 4289409513ull, 4289680569ull, 4289938406ull,
    4290183668ull, 4290416968ull, 4290638890ull, 4290849989ull, 4291050792ull,
    4291241802ull, 4291423497ull, 4291596330ull, 4291760734ull, 4291917120ull,
    4292065879ull, 4292207382ull, 4292341985ull, 4292470023ull, 4292591816ull,
    4292707670ull, 4292817873ull, 4292922702ull, 4293022418ull, 4293117270ull,
    4293207497ull, 4293293324ull, 4293374964ull, 4293452623ull, 4293526494ull,
    4293596763ull, 4293663605ull, 4293727187ull, 4293787667ull, 4293845199ull,
    4293899924ull, 4293951980ull, 4294001498ull, 4294048600ull, 4294093406ull,
    4294136026ull, 4294176567ull, 4294215131ull, 4294251815ull, 4294286709ull,
    4294319902ull, 4294351476ull, 4294381510ull, 4294410079ull, 4294437254ull,
    4294463105ull, 4294487695ull, 4294511085ull, 4294533335ull, 4294554499ull,
    4294574631ull, 4294593782ull, 4294611998ull, 4294629326ull, 4294645809ull,
    4294661488ull, 4294676403ull, 4294690590ull, 4294704085ull, 4294716922ull,
    4294729133ull, 4294740748ull, 4294751797ull, 4294762307ull, 4294772304ull,
    4294781814ull, 4294790860ull, 4294799465ull, 4294807650ull, 4294815436ull,
    4294822842ull, 4294829888ull, 4294836589ull, 4294842964ull, 4294849027ull,
    4294854795ull, 4294860282ull, 4294865501ull, 4294870466ull, 4294875188ull,
    4294879680ull, 4294883953ull, 4294888018ull, 4294891884ull, 4294895562ull,
    4294899061ull, 4294902389ull, 4294905554ull, 4294908565ull, 4294911430ull,
    4294914154ull, 4294916746ull, 4294919211ull, 4294921556ull, 4294923787ull,
    4294925909ull, 4294927927ull, 4294929847ull, 4294931674ull, 4294933411ull,
    4294935064ull, 4294936636ull, 4294938131ull, 4294939553ull, 4294940906ull,
    4294942193ull, 4294943418ull, 4294944582ull, 4294945690ull, 4294946744ull,
    4294947746ull, 4294948699ull, 4294949606ull, 4294950469ull, 4294951290ull,
    4294952070ull, 4294952813ull, 4294953519ull, 4294954191ull, 4294954830ull,
    4294967296ull,
};

/* Clipped-exponential integers in [0, 255] (SIFT-descriptor-like): the value is the
 * smallest x with u < T[x], u the top 32 bits of stream element e. */
void px_gen_sift(uint64_t seed, int64_t start, int64_t count, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < count; ++e) {
        uint64_t u = stream_at(seed, (uint64_t)(start + e)) >> 32;
        int lo = 0, hi = 255; /* smallest x in [0,255] with u < T[x]; T[255] = 2^32 > u */
        while (lo < hi) {
            int mid = (lo + hi) >> 1;
            if (u < k_sift_thresholds[mid]) hi = mid; else lo = mid + 1;
        }
        out[e] = (float)lo;
    }
}

/* Row-wise unit normalisation: x / sqrt(sum x^2) with a sequential f32 sum and
 * IEEE sqrt and divide (build with -ffp-contract=off). Zero rows are left as is. */
void px_gen_normalize_rows(float* x, int64_t rows, int64_t dim) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float* v = x + r * dim;
        float s = 0.0f;
        for (int64_t d = 0; d < dim; ++d) s = s + v[d] * v[d];
        float nrm = sqrtf(s);
        if (nrm > 0.0f)
            for (int64_t d = 0; d < dim; ++d) v[d] = v[d] / nrm;
    }
}

/* Bernoulli(p) keep-mask: element e kept iff (top 32 bits of stream element e) < p * 2^32. */
void px_gen_mask(uint64_t seed, int64_t start, int64_t count, double p, uint8_t* out) {
    uint64_t thr = p <= 0.0 ? 0 : (p >= 1.0 ? (1ull << 32) : (uint64_t)(p * 4294967296.0));
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < count; ++e)
        out[e] = (uint8_t)((stream_at(seed, (uint64_t)(start + e)) >> 32) < thr);
}

int px_gen_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
