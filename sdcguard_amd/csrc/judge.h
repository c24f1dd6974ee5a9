// The scoring arithmetic of one (row, block) pair, shared by every kernel that scores block checksums.
//
// judge_serve: the serving check's two checksums of a pair (_serve_fast.py:334-402, `_judge`; serve.py:301-396):
//   unjudged checksums score 0 and are counted.
// judge_one: one checksum of the training check (checksum.py:435-530 `_zscores` with `_judge_nonfinite` :359-383):
//   unjudged checksums score -1.
// Both take the check's constants from an argument struct with the fields u (unit roundoff), h (half the subnormal
// spacing), abs_floor, l1c (l1_floor_coef(k)), zt (the line), lim_a (largest finite output), capk (the "impossible"
// factor) and, for judge_serve, lim_big.
#pragma once
#include "blocksums.h"

struct PairScore {
  float z0, z1;
  float zc, dc;
  bool sec;
  int unk;
};

// _serve_fast.py:334-402 (`_judge`) for one (row, block) pair, serving flavour (unjudged checksums score 0).
template <class A>
__device__ __forceinline__ PairScore judge_serve(float plain, float sgn, float sq, float l1, float xn, float asum,
                                                 float e0, float e1, float sc0, float sc1, float bs0, float bs1,
                                                 float bmaxv, float bmbv, float b2n0, float b2n1, float b2m0,
                                                 float b2m1, float wf, const A& a) {
  const float inf = __builtin_inff();
  const float nanv = __builtin_nanf("");
  float exp0 = e0 * sc0 + bs0;
  float exp1 = e1 * sc1 + bs1;
  float bound = asum * bmaxv + bmbv;
  float rsq = fsqrt(sq);
  float noise = rsq * a.u;
  float fl0 = xn * b2n0 * 1e-5f;
  float fl1 = xn * b2n1 * 1e-5f;
  float hl0 = asum * b2m0 * a.l1c;
  float hl1 = asum * b2m1 * a.l1c;
  fl0 = fminf(fabsf(fl0) < inf ? fl0 : inf, fabsf(hl0) < inf ? hl0 : inf);
  fl1 = fminf(fabsf(fl1) < inf ? fl1 : inf, fabsf(hl1) < inf ? hl1 : inf);
  const float bigfl = bound * (float)(1e-5 * 128.0);
  fl0 = fl0 < inf ? fl0 : bigfl;
  fl1 = fl1 < inf ? fl1 : bigfl;
  float swf = fsqrt(wf);
  float tail = a.abs_floor + swf * a.h;
  float den0 = (noise + fl0) + tail;
  float den1 = (noise + fl1) + tail;
  float d0 = fabsf(exp0 - plain);
  float d1 = fabsf(exp1 - sgn);
  float z0 = fdiv(d0, den0);
  float z1 = fdiv(d1, den1);
  float worst = (l1 * (1.25f * a.u) + (1.25f * a.h * wf)) + fl0 + a.abs_floor;
  float zw = fdiv(d0, worst) * a.zt;
  z0 = (z0 == z0 && zw == zw) ? fminf(z0, zw) : nanv;
  float lim = bound * 1.01f;
  bool nfin = !(noise < inf);
  bool e_bad0 = !(fabsf(exp0) < inf);
  bool a_bad0 = !e_bad0 && !(fabsf(plain) < inf);
  bool big0 = nfin && !e_bad0 && !a_bad0;
  bool nan0 = !(z0 == z0);
  z0 = z0 == z0 ? z0 : 0.f;
  z0 = e_bad0 ? 0.f : z0;
  float cap = bound * a.capk + 2.0f * a.h;
  bool imposs = !nfin && (lim < a.lim_big) && (rsq > cap * swf);
  bool ok_a = lim < a.lim_a, ok_big = lim < a.lim_big;
  z0 = (imposs && !e_bad0 && !a_bad0) ? inf : z0;
  z0 = a_bad0 ? (ok_a ? inf : 0.f) : z0;
  z0 = big0 ? (ok_big ? inf : 0.f) : z0;
  bool e_bad1 = !(fabsf(exp1) < inf);
  bool a_bad1 = !e_bad1 && !(fabsf(sgn) < inf);
  bool big1 = nfin && !e_bad1 && !a_bad1;
  bool nan1 = !(z1 == z1);
  z1 = z1 == z1 ? z1 : 0.f;
  z1 = e_bad1 ? 0.f : z1;
  z1 = (imposs && !e_bad1 && !a_bad1) ? inf : z1;
  z1 = a_bad1 ? (ok_a ? inf : 0.f) : z1;
  z1 = big1 ? (ok_big ? inf : 0.f) : z1;
  bool unk0 = (nan0 && !imposs && !a_bad0 && !big0) || e_bad0 || (a_bad0 && !ok_a) || (big0 && !ok_big);
  bool unk1 = (nan1 && !imposs && !a_bad1 && !big1) || e_bad1 || (a_bad1 && !ok_a) || (big1 && !ok_big);
  PairScore r;
  r.z0 = z0;
  r.z1 = z1;
  r.sec = z1 > z0;
  r.zc = r.sec ? z1 : z0;
  r.dc = r.sec ? (a_bad1 ? nanv : den1) : (a_bad0 ? nanv : den0);
  r.unk = (int)unk0 + (int)unk1;
  return r;
}


// one checksum of checksum._zscores + _judge_nonfinite (unjudged = -1)
template <class A>
__device__ __forceinline__ float judge_one(float expected, float actual, float noise, float cn, float fl, float bound,
                                           float wf, float l1, bool plain, const A& a, float& den) {
  const float inf = __builtin_inff();
  const float swf = fsqrt(wf);
  den = (noise + fl) + (a.abs_floor + swf * a.h);
  const float diff = fabsf(expected - actual);
  float z = fdiv(diff, den);
  if (plain) {
    const float worst = ((l1 * (1.25f * a.u) + 1.25f * wf * a.h) + fl) + a.abs_floor;
    const float zw = fdiv(diff, worst) * a.zt;
    z = (z == z && zw == zw) ? fminf(z, zw) : __builtin_nanf("");
  }
  const bool e_bad = !(fabsf(expected) < inf);
  const bool a_bad = !(fabsf(actual) < inf) && !e_bad;
  const bool big = !(noise < inf) && !e_bad && !a_bad;
  const float lim = bound * 1.01f;
  z = z == z ? z : -1.f;
  z = e_bad ? -1.f : z;
  const float cap = bound * a.capk + 2.f * a.h;
  const bool imposs = !e_bad && !a_bad && !big && (lim < 1e18f) && (cn > cap * swf);
  z = imposs ? inf : z;
  z = a_bad ? (lim < a.lim_a ? inf : -1.f) : z;
  z = big ? (lim < 1e18f ? inf : -1.f) : z;
  return z;
}


// The same two scores where every input is finite and the pair is not "impossible" (the common case): ok tells
// whether that held; where it did, the result is judge_serve's (the same expressions, without its non-finite
// selects), else the caller takes judge_serve.
template <class A>
__device__ __forceinline__ PairScore judge_serve_clean(float plain, float sgn, float sq, float l1, float xn,
                                                       float asum, float e0, float e1, float sc0, float sc1,
                                                       float bs0, float bs1, float bmaxv, float bmbv, float b2n0,
                                                       float b2n1, float b2m0, float b2m1, float wf, const A& a,
                                                       bool& ok) {
  const float inf = __builtin_inff();
  const float exp0 = e0 * sc0 + bs0;
  const float exp1 = e1 * sc1 + bs1;
  const float bound = asum * bmaxv + bmbv;
  const float rsq = fsqrt(sq);
  const float noise = rsq * a.u;
  float fl0 = xn * b2n0 * 1e-5f;
  float fl1 = xn * b2n1 * 1e-5f;
  const float hl0 = asum * b2m0 * a.l1c;
  const float hl1 = asum * b2m1 * a.l1c;
  fl0 = fminf(fabsf(fl0) < inf ? fl0 : inf, fabsf(hl0) < inf ? hl0 : inf);
  fl1 = fminf(fabsf(fl1) < inf ? fl1 : inf, fabsf(hl1) < inf ? hl1 : inf);
  const float bigfl = bound * (float)(1e-5 * 128.0);
  fl0 = fl0 < inf ? fl0 : bigfl;
  fl1 = fl1 < inf ? fl1 : bigfl;
  const float swf = fsqrt(wf);
  const float tail = a.abs_floor + swf * a.h;
  const float den0 = (noise + fl0) + tail;
  const float den1 = (noise + fl1) + tail;
  const float d0 = fabsf(exp0 - plain);
  const float d1 = fabsf(exp1 - sgn);
  float z0 = fdiv(d0, den0);
  const float z1 = fdiv(d1, den1);
  const float worst = (l1 * (1.25f * a.u) + (1.25f * a.h * wf)) + fl0 + a.abs_floor;
  const float zw = fdiv(d0, worst) * a.zt;
  const float lim = bound * 1.01f;
  const float cap = bound * a.capk + 2.0f * a.h;
  // d finite <=> expected and actual finite; noise finite; no NaN score; not "impossible"
  ok = (d0 < inf) && (d1 < inf) && (noise < inf) && (z0 == z0) && (zw == zw) && (z1 == z1) &&
       !((lim < a.lim_big) && (rsq > cap * swf));
  z0 = fminf(z0, zw);
  PairScore r;
  r.z0 = z0;
  r.z1 = z1;
  r.sec = z1 > z0;
  r.zc = r.sec ? z1 : z0;
  r.dc = r.sec ? den1 : den0;
  r.unk = 0;
  return r;
}

// judge_one where the checksum's inputs are finite and it is not "impossible": ok tells whether that held; where it
// did, the score is judge_one's.
template <class A>
__device__ __forceinline__ float judge_one_clean(float expected, float actual, float noise, float cn, float fl,
                                                 float bound, float wf, float l1, bool plain, const A& a, float& den,
                                                 bool& ok) {
  const float inf = __builtin_inff();
  const float swf = fsqrt(wf);
  den = (noise + fl) + (a.abs_floor + swf * a.h);
  const float diff = fabsf(expected - actual);
  float z = fdiv(diff, den);
  bool fin = z == z;
  if (plain) {
    const float worst = ((l1 * (1.25f * a.u) + 1.25f * wf * a.h) + fl) + a.abs_floor;
    const float zw = fdiv(diff, worst) * a.zt;
    fin = fin && (zw == zw);
    z = fminf(z, zw);
  }
  const float lim = bound * 1.01f;
  const float cap = bound * a.capk + 2.f * a.h;
  ok = (diff < inf) && (noise < inf) && fin && !((lim < 1e18f) && (cn > cap * swf));
  return z;
}
