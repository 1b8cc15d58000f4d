# SPDX-License-Identifier: BSD-3-Clause
"""Sample optimizers of `loop-explore --search iterative`
(src/xtc/search/optimizers.py:20-236, interface src/xtc/itf/search/optimizer.py).

An optimizer proposes the next batch of strategy samples and learns from the
measured results.  The measure it maximises is the fraction of peak,
peak_time / time (0 for a failed sample), as the reference's explorer feeds
it (src/xtc/search/explore.py:515-538).

  * "random": every batch is `batch` fresh samples of the strategy.
  * "random-forest-{default,explore,aggressive}": until `update_first`
    samples are observed, `batch` picks (with replacement) among
    `batch_candidates` fresh samples; then a random-forest regressor over the
    sample vectors scores the candidates with an upper confidence bound,
    mean - best + beta_t * std over the trees, beta_t = max(0.05,
    beta / n_observed^alpha), and the `batch` best are proposed.  The forest
    is refit after `update_first` observations and then every
    `update_period` more (both default to the batch size).

The names, presets, the sampling seeds (one draw from random.Random(seed)
per proposal) and the YAML override file of `--optimizer-config` are kept as
in the reference so that a seeded run proposes the same schedules.
"""

from __future__ import annotations

import logging
import random
from typing import Any, Callable, Iterator, Sequence

import numpy as np

__all__ = ["Optimizer", "RandomOptimizer", "RandomForestOptimizer", "Optimizers"]

Sample = list[int]
SampleFn = Callable[[int, int], Iterator[Sequence[int]]]

logger = logging.getLogger("xtc_amd.search.optimizers")


class Optimizer:
    """suggest() -> next batch; observe(x, y) after it ran; finished()."""

    def __init__(self, sample_fn: SampleFn, batch: int, seed: int, **_: Any) -> None:
        self.sample_fn = sample_fn
        self.batch = int(batch)
        self.rng = random.Random(seed)

    def _fresh(self, n: int) -> list[Sample]:
        return [list(x) for x in self.sample_fn(n, self.rng.randint(0, 2**32 - 1))]

    def suggest(self) -> list[Sample]:
        raise NotImplementedError

    def observe(self, x: list[Sample], y: list[float]) -> None:
        pass

    def finished(self) -> None:
        pass


class RandomOptimizer(Optimizer):
    def suggest(self) -> list[Sample]:
        return self._fresh(self.batch)


class RandomForestOptimizer(Optimizer):
    def __init__(
        self,
        sample_fn: SampleFn,
        batch: int,
        seed: int,
        batch_candidates: int,
        beta: float,
        alpha: float,
        update_first: int | None,
        update_period: int | None,
        n_estimators: int,
        max_depth: int,
        min_samples_leaf: int,
        max_features: float,
    ) -> None:
        from sklearn.ensemble import RandomForestRegressor

        super().__init__(sample_fn, batch, seed)
        self.batch_candidates = int(batch_candidates)
        self.beta = float(beta)
        self.alpha = float(alpha)
        self.beta_floor = 0.05
        self.update_first = int(update_first or batch)
        self.update_period = int(update_period or batch)
        self.fitted_on = 0
        self.X: list[Sample] = []
        self.y: list[float] = []
        self.best_x: Sample = []
        self.best_y = 0.0
        self.last_beta: float | None = None
        self.forest = RandomForestRegressor(
            n_estimators=n_estimators,
            max_depth=max_depth,
            min_samples_leaf=min_samples_leaf,
            min_samples_split=2 * min_samples_leaf,
            max_features=max_features,
            random_state=seed,
            n_jobs=1,
        )
        self.history: list[str] = []

    def acquisition(self, candidates: list[Sample]) -> np.ndarray:
        """Upper confidence bound of each candidate's improvement."""
        per_tree = np.stack([tree.predict(candidates) for tree in self.forest.estimators_])
        beta = max(self.beta_floor, self.beta / (len(self.y) ** self.alpha))
        self.last_beta = beta
        return (per_tree.mean(axis=0) - self.best_y) + beta * per_tree.std(axis=0)

    def suggest(self) -> list[Sample]:
        candidates = self._fresh(self.batch_candidates)
        if len(self.X) < self.update_first:
            return self.rng.choices(candidates, k=self.batch)
        scores = self.acquisition(candidates)
        top = np.argpartition(scores, -self.batch)[-self.batch :]
        return [candidates[i] for i in top]

    def observe(self, x: list[Sample], y: list[float]) -> None:
        self.X.extend(list(v) for v in x)
        self.y.extend(float(v) for v in y)
        for xi, yi in zip(x, y):
            if yi > self.best_y:
                self.best_x, self.best_y = list(xi), float(yi)
        self.history.append(f"after {len(self.X)} points: best {self.best_y}, batch {list(y)}, ucb beta {self.last_beta}")
        if len(self.X) < self.update_first:
            return
        n = self.update_first + (len(self.X) - self.update_first) // self.update_period * self.update_period
        if n > self.fitted_on:
            self.forest.fit(self.X[:n], self.y[:n])
            self.fitted_on = n

    def finished(self) -> None:
        logger.info("optimizer finished: best %s (%.4g of peak)", self.best_x, self.best_y)
        for line in self.history:
            logger.debug(line)


class _Preset:
    """An optimizer class with preset keyword arguments, overridable by a
    YAML file (`--optimizer-config`)."""

    def __init__(self, cls: type[Optimizer], preset: dict[str, Any]) -> None:
        self.cls = cls
        self.preset = preset

    def __call__(self, sample_fn: SampleFn, batch: int, seed: int, config_file: str = "") -> Optimizer:
        kwargs = dict(self.preset)
        if config_file:
            import yaml

            with open(config_file) as f:
                kwargs.update(yaml.safe_load(f) or {})
        return self.cls(sample_fn, batch, seed, **kwargs)


def _forest(**kw: Any) -> dict[str, Any]:
    return {"batch_candidates": 1000, "update_first": None, "update_period": None, "n_estimators": 300, **kw}


class Optimizers:
    _map: dict[str, _Preset] = {
        "random": _Preset(RandomOptimizer, {}),
        "random-forest-explore": _Preset(
            RandomForestOptimizer,
            _forest(beta=5, alpha=0.6, max_depth=10, min_samples_leaf=3, max_features=0.9),
        ),
        "random-forest-default": _Preset(
            RandomForestOptimizer,
            _forest(beta=2.5, alpha=0.7, max_depth=12, min_samples_leaf=5, max_features=0.8),
        ),
        "random-forest-aggressive": _Preset(
            RandomForestOptimizer,
            _forest(beta=2, alpha=0.8, n_estimators=200, max_depth=8, min_samples_leaf=5, max_features=0.7),
        ),
    }

    @classmethod
    def names(cls) -> list[str]:
        return list(cls._map)

    @classmethod
    def from_name(cls, name: str) -> _Preset:
        if name not in cls._map:
            raise ValueError(f"unknown optimizer name: {name} (one of {', '.join(cls._map)})")
        return cls._map[name]
