/* CPU oracle (test infrastructure only): the layer boundary around the token
 * mixers, Ops.AddInPlace (src/Qwen35Sharp.Model/Ops.cs:677-710) and
 * Qwen35Ops.RmsNormZeroCentered (src/Qwen35Sharp.Model/Qwen35Ops.cs:22-64),
 * as Qwen35Model.DecodeBlock chains them (Qwen35Model.Decode.cs:226-235). */
#include <math.h>

#include "q35_oracle.h"

/* VecDotQ4K.HorizontalSum (VecDotQ4K.cs:145-151) of the 8 lanes. */
static float hsum8_lanes(const float* a) {
    return ((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]));
}

/* hidden += delta (when delta is non-null; fp32 adds), then per row y =
 * (h * scale) * (1 + w) with scale = 1 / sqrt(sum / dim + eps), sum of
 * squares over 8 fp32 FMA lanes (lane l takes elements l, l + 8, ...) for
 * the whole 8-element groups, their horizontal sum, and then the dim % 8 tail
 * elements one at a time (square rounded, then added).  w null means 0. */
void q35o_add_rmsnorm(float* hidden, const float* delta, const float* w, float* y, int dim, int rows,
                      float eps) {
    for (int r = 0; r < rows; r++) {
        float* h = hidden + (long)r * dim;
        if (delta)
            for (int i = 0; i < dim; i++) h[i] = h[i] + delta[(long)r * dim + i];
        float acc[8] = {0};
        int i = 0;
        for (; i <= dim - 8; i += 8)
            for (int l = 0; l < 8; l++) acc[l] = fmaf(h[i + l], h[i + l], acc[l]);
        float sum = hsum8_lanes(acc);
        for (; i < dim; i++) {
            const float sq = h[i] * h[i];
            sum = sum + sq;
        }
        const float scale = 1.0f / sqrtf(sum / (float)dim + eps);
        for (int k = 0; k < dim; k++) {
            const float t = h[k] * scale;
            y[(long)r * dim + k] = t * (1.0f + (w ? w[k] : 0.0f));
        }
    }
}
