/* Sampler behind synth.gen_c4 (a first-order Markov byte source): with
 * row-wise cumulative transition probabilities cum[256][256] and uniforms
 * u[0..n), byte t is the chain state x_t and x_{t+1} is the first index i
 * with cum[x_t][i] >= u[t] (numpy's searchsorted, side "left"), clamped to
 * 255.  Returns the state after the last byte so blocks can be chained. */
#include <stddef.h>
#include <stdint.h>

int synth_markov_fill(const double* cum, const double* u, int64_t n, int x0, uint8_t* out) {
    int x = x0;
    for (int64_t t = 0; t < n; ++t) {
        out[t] = (uint8_t)x;
        const double* row = cum + (size_t)x * 256;
        const double v = u[t];
        int lo = 0, hi = 256;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (row[mid] < v) lo = mid + 1;
            else hi = mid;
        }
        x = lo > 255 ? 255 : lo;
    }
    return x;
}
