// k_mel.hip — log-mel front-end on the GPU (transcribe.c:177-214).
//
// Per frame t of a clip: samples [t*160, t*160+400) of the zero-padded
// (200 each side), pre-emphasised (x[i] - 0.97 x[i-1]) signal, Hann window,
// 512-point FFT, power spectrum (257 bins), 128 Slaney mel filters,
// log(x + 2^-24).  Then each mel bin is normalised over the clip's frames
// with mean and var/(T-1).  One workgroup transforms one frame in LDS
// (radix-2, twiddles from a host table); a second kernel normalises rows.
#include "ct_dev.h"
#include "ct_launch.h"
#include "../../include/model_types.h"

namespace {

constexpr int NF = N_FFT;   // 512

__global__ __launch_bounds__(256) void mel_frames_kernel(float *mel,
                                                         const CtMelClip *clips, const int *frame_clip,
                                                         const float *hann, const float *twr,
                                                         const float *twi, const float *fb,
                                                         const int *fb_lo, const int *fb_hi) {
    __shared__ float re[NF], im[NF], ps[N_BINS];
    const int f = blockIdx.x;
    const CtMelClip c = clips[frame_clip[f]];
    const int t = f - c.frame0;
    const int tid = threadIdx.x;
    const int off = t * HOP_LEN;
    const int pad = WIN_LEN / 2;
    // load windowed, pre-emphasised samples in bit-reversed order
    for (int j = tid; j < NF; j += 256) {
        float v = 0.0f;
        if (j < WIN_LEN) {
            const int a = off + j - pad;              // index into the clip
            const float x1 = (a >= 0 && a < c.n) ? c.pcm[a] : 0.0f;
            const float x0 = (a - 1 >= 0 && a - 1 < c.n && off + j > 0) ? c.pcm[a - 1] : 0.0f;
            v = (x1 - 0.97f * x0) * hann[j];
        }
        const int r = __brev((unsigned)j) >> (32 - 9);
        re[r] = v;
        im[r] = 0.0f;
    }
    __syncthreads();
    for (int half = 1; half < NF; half <<= 1) {
        const int k = tid;                         // 256 butterflies per stage
        const int grp = k / half, pos = k % half;
        const int i0 = grp * 2 * half + pos, i1 = i0 + half;
        const int tw = pos * (NF / (2 * half));
        const float wr = twr[tw], wi = twi[tw];
        const float vr = re[i1] * wr - im[i1] * wi;
        const float vi = re[i1] * wi + im[i1] * wr;
        const float ur = re[i0], ui = im[i0];
        __syncthreads();
        re[i0] = ur + vr; im[i0] = ui + vi;
        re[i1] = ur - vr; im[i1] = ui - vi;
        __syncthreads();
    }
    for (int i = tid; i < N_BINS; i += 256) ps[i] = re[i] * re[i] + im[i] * im[i];
    __syncthreads();
    if (tid < N_MELS) {
        float acc = 0.0f;
        for (int i = fb_lo[tid]; i < fb_hi[tid]; i++) acc += fb[tid * N_BINS + i] * ps[i];
        mel[c.mel0 + (long)tid * c.T + t] = logf(acc + 5.9604644775390625e-8f);
    }
}

__global__ __launch_bounds__(64) void mel_norm_kernel(float *mel, const CtMelClip *clips) {
    const CtMelClip c = clips[blockIdx.y];
    const int m = blockIdx.x, lane = threadIdx.x;
    float *row = mel + c.mel0 + (long)m * c.T;
    float s = 0.0f;
    for (int t = lane; t < c.T; t += 64) s += row[t];
    const float mu = wave_sum(s) / (float)c.T;
    float q = 0.0f;
    for (int t = lane; t < c.T; t += 64) { const float d = row[t] - mu; q += d * d; }
    const float var = wave_sum(q) / (float)(c.T - 1);
    const float r = 1.0f / sqrtf(var + 1e-5f);
    for (int t = lane; t < c.T; t += 64) row[t] = (row[t] - mu) * r;
}

}  // namespace

extern "C" void ctk_mel(float *mel, const CtMelClip *clips, int n_clips,
                        const int *frame_clip, int n_frames, const CtMelTables *tab, hipStream_t s) {
    if (n_frames <= 0) return;
    hipLaunchKernelGGL(mel_frames_kernel, dim3(n_frames), dim3(256), 0, s, mel, clips, frame_clip,
                       tab->hann, tab->twr, tab->twi, tab->fb, tab->fb_lo, tab->fb_hi);
    hipLaunchKernelGGL(mel_norm_kernel, dim3(N_MELS, n_clips), dim3(64), 0, s, mel, clips);
}
